"""Keys with a resident dense `a` (pcx_keys_resident_a; crates/pc-gpu/src/ks.rs:408-411, 1259-1262: a group that stores
`a` regenerates its digits below regen_digits and reads the rest): every regen_digits from the full regeneration down
to none gives the same words, since the resident rows are the KSKA expander's own. Checked through the fast dot (the
retry table for the regenerated digits), the table-only path (the kernel table's ks_dot_key), the summed rotations and
a batched relinearized product with rescale, at the C3 shape (31-bit primes) and at N = 2^12."""
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


def random_ct(ch, top, rng, k=1):
    ct = np.zeros((k, 2, ch.rows, ch.n), np.uint32)
    for c in range(k):
        for part in range(2):
            for t in range(top + 1):
                ct[c, part, t] = rng.integers(0, ch.primes[t], ch.n)
    return ct


@pytest.mark.parametrize("name,top", [("c3", 29), ("c3", 14), ("small", 5)])
def test_resident_digits_give_the_same_words(stream, name, top):
    ch = pa.preset(name)
    ctx = pa.Context(ch, k_rot=6, k_max=2)
    rng = np.random.default_rng(top)
    steps = [1, 2, 3, 5, 8, 64]
    gals = [twin.rotation_galois(s, ch.n) for s in steps]
    drbg = pa.Drbg([7, 7, 7, 7, 1, 2, 3, top], 0)
    secret = drbg.sparse_ternary(ch.n, 64)
    seeds, errors = drbg.keygen_draw(len(gals), ch.dnum, ch.n)
    keys = pa.Keys(ctx, gals, seeds=seeds, secret=secret, errors=errors)
    rseed, rerr = drbg.keygen_draw(1, ch.dnum, ch.n)
    relin = pa.Keys(ctx, [1], seeds=rseed, secret=secret, errors=rerr, relin=True)
    x = pa.DevBuf.from_array(random_ct(ch, top, rng)[0])
    a2 = pa.DevBuf.from_array(random_ct(ch, top, rng, 2))
    b2 = pa.DevBuf.from_array(random_ct(ch, top, rng, 2))
    outs = ctx.ct_buf(len(gals))
    one, summed, prod = ctx.ct_buf(), ctx.ct_buf(), ctx.ct_buf(2)
    R = ch.rows

    def run():
        outs.zero()
        ctx.rotate_hoisted(keys, list(range(len(gals))), x, top, outs, stream)
        ctx.rotate(keys, 4, x, top, one, stream)
        ctx.rotate_sum(keys, [0, 1, 2, 3], x, top, summed, stream)
        ctx.mul_relin_rescale(relin, a2, b2, top, prod, stream, K=2)
        stream.sync()
        return (outs.download((len(gals), 2, R, ch.n))[:, :, : top + 1], one.download((2, R, ch.n))[:, : top + 1],
                summed.download((2, R, ch.n))[:, : top + 1], prod.download((2, 2, R, ch.n))[:, :, : top - 1])

    say(f"[resident a] {name} top={top}: every digit regenerated")
    want = run()
    for regen in (2, 1, 0):
        keys.resident_a(regen, stream)
        relin.resident_a(regen, stream)
        say(f"[resident a] {name} top={top}: digits >= {regen} resident")
        got = run()
        for g, w, what in zip(got, want, ("hoisted", "rotate", "sum", "product")):
            assert (g == w).all(), (regen, what)
        prev = ctx.table_only(True)
        say(f"[resident a] {name} top={top}: digits >= {regen} resident, kernel table only")
        got = run()
        ctx.table_only(prev)
        for g, w, what in zip(got, want, ("hoisted", "rotate", "sum", "product")):
            assert (g == w).all(), (regen, what, "table")
    assert keys.resident_bytes() == len(gals) * ch.dnum * R * ch.n * 4
    keys.resident_a(ch.dnum, stream)  # every digit regenerated again
    assert all((g == w).all() for g, w in zip(run(), want))
    with pytest.raises(pa.HipError):
        keys.resident_a(-1, stream)
