"""pcx_rotate_and_sum_noalloc (the ladder with its scratch ciphertext in the library's static device array) against
pcx_rotate_and_sum with a caller's scratch, word for word, through the C-ABI: two calls in a row on the C3 chain, the
second at a lower limb top (a smaller input that reuses the array the first left full), rung by rung so that every
rotation goes through the scratch, then a radix-4 ladder on a second, smaller ring; and the refusal of a rung wider
than 8 bits. Each step prints its case before the GPU runs."""
import sys

import numpy as np
import pytest

import perseus_amd as pa
from perseus_amd._lib import LIB
from tests import twin

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def random_ct(ch, top, seed):
    rng = np.random.default_rng(seed)
    ct = np.zeros((2, ch.rows, ch.n), np.uint32)
    for part in range(2):
        for t in range(top + 1):
            ct[part, t] = rng.integers(0, ch.primes[t], ch.n)
    return ct


def keys_for(ch, ctx, steps, seed):
    oc = twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum)
    g = twin.Prng([seed, 9, 8, 7, 6, 5, 4, 3], 0)
    s_eval = oc.secret_eval(g.sparse_ternary(ch.n, 192))
    gals = [twin.rotation_galois(r, ch.n) for r in steps]
    ks = [oc.rotation_key(g, s_eval, x) for x in gals]
    return pa.Keys(ctx, gals, seeds=np.stack([k[0] for k in ks]), b=[k[1] for k in ks], bits=0)


def both(ch, ctx, keys, st, top, start, stop, radix, seed):
    ct = random_ct(ch, top, seed)
    x = pa.DevBuf.from_array(ct)
    want_buf, tmp, got_buf = ctx.ct_buf(), ctx.ct_buf(), ctx.ct_buf()
    assert LIB.pcx_rotate_and_sum(ctx.h, keys.h, x.addr(), top, start, stop, radix, want_buf.addr(), tmp.addr(),
                                  st.h) == 0
    assert LIB.pcx_rotate_and_sum_noalloc(ctx.h, keys.h, x.addr(), top, start, stop, radix, got_buf.addr(),
                                          st.h) == 0
    st.sync()
    want = want_buf.download((2, ch.rows, ch.n))
    got = got_buf.download((2, ch.rows, ch.n))
    assert (got[:, : top + 1] == want[:, : top + 1]).all()


def test_noalloc_ladder_equals_the_ladder():
    assert pa.device_count() >= 1, "no GPU visible"
    twin.set_threads(16)
    st = pa.Stream()
    ch = pa.preset("c3")
    ctx = pa.Context(ch, k_rot=4)
    assert ctx.ct_words <= LIB.pcx_ct_words(ctx.h) <= 2 * 64 * 65536
    keys = keys_for(ch, ctx, [1, 2, 3, 4, 8, 12], 71)
    say("[noalloc] c3 top 29, steps 1..15 rung by rung (every rotation through the scratch)")
    both(ch, ctx, keys, st, 29, 1, 16, 1, 5)
    say("[noalloc] c3 top 13 (smaller input, the array left full by the first call), rung by rung")
    both(ch, ctx, keys, st, 13, 1, 16, 1, 6)
    say("[noalloc] small ring N=2^12 top 5, radix 4 (summed rungs) and rung by rung")
    chs = pa.preset("small")
    ctxs = pa.Context(chs, k_rot=4)
    keys_s = keys_for(chs, ctxs, [1, 2, 3, 4, 8, 12], 72)
    both(chs, ctxs, keys_s, st, 5, 1, 16, 2, 7)
    both(chs, ctxs, keys_s, st, 3, 1, 8, 1, 8)
    say("[noalloc] a rung of 9 bits is refused (-2), before any GPU work")
    x = ctxs.ct_buf()
    assert LIB.pcx_rotate_and_sum_noalloc(ctxs.h, keys_s.h, x.addr(), 5, 1, 1 << 10, 9, x.addr(), st.h) == -2


def test_noalloc_ladder_in_a_captured_graph():
    """The entry point under stream capture (its scratch address taken at context creation): the ladder captured into
    one HIP graph, replayed three times with a new input uploaded and eager work between the replays; every replay
    equals pcx_rotate_and_sum run eagerly on the same input."""
    assert pa.device_count() >= 1, "no GPU visible"
    st = pa.Stream()
    ch = pa.preset("small")
    ctx = pa.Context(ch, k_rot=4)
    keys = keys_for(ch, ctx, [1, 2, 3, 4, 8, 12], 73)
    top = 5
    x, got_buf = ctx.ct_buf(), ctx.ct_buf()
    say("[noalloc] small ring top 5: the ladder (1..16, radix 4) captured into a graph")

    def work():
        assert LIB.pcx_rotate_and_sum_noalloc(ctx.h, keys.h, x.addr(), top, 1, 16, 2, got_buf.addr(), st.h) == 0

    x.upload(random_ct(ch, top, 90), st)
    g = pa.Graph(st, work)
    want_buf, tmp = ctx.ct_buf(), ctx.ct_buf()
    for rep in range(3):
        say(f"[noalloc] graph replay {rep}")
        ct = random_ct(ch, top, 91 + rep)
        x.upload(ct, st)
        got_buf.zero()
        g.launch(st)
        st.sync()
        got = got_buf.download((2, ch.rows, ch.n))
        assert LIB.pcx_rotate_and_sum(ctx.h, keys.h, x.addr(), top, 1, 16, 2, want_buf.addr(), tmp.addr(),
                                      st.h) == 0
        st.sync()
        want = want_buf.download((2, ch.rows, ch.n))
        assert (got[:, : top + 1] == want[:, : top + 1]).all(), rep
