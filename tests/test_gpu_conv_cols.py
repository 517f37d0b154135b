"""The conversions streamed into the forward NTT's column pass (pch::conv_cols: the ModUp of every digit, the ModDown
over more special primes than the register-held fused form takes, and the ModDown-rescale's exact conversion of
kp + 2 sources) against the plan's bconv then ntt_fwd, word for word, through the C-ABI: the same context runs each
operation with pcx_ctx_conv_fusion on (7) and off (0). Chains: C5 (30-bit primes, Harvey butterflies, 16 special
primes, digits of 16 limbs), C3 (31-bit primes: non-lazy butterflies, and products whose sums fold to a residue
every 4 sources), and N = 2^12 / 2^14 chains of 16 special primes (other column-pass shapes); tops that leave a
partial digit, a single limb, and K = 2 ciphertexts. The fused path against the oracle is covered by the rotation,
product and bootstrap tests, which run it by default."""
import sys

import numpy as np
import pytest

import perseus_amd as pa
from perseus_amd.chains import make
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


_SETUP = {}


def setup(name):
    if name not in _SETUP:
        if name == "t12":
            ch = make("t12", 12, 20, 16, 3, 30)
        elif name == "t14":
            ch = make("t14", 14, 26, 16, 3, 30)
        else:
            ch = pa.preset(name)
        ctx = pa.Context(ch, k_rot=2, k_max=2)
        rng = np.random.default_rng(len(name) * 7 + ch.logn)
        s = rng.integers(-1, 2, ch.n).astype(np.int8)
        gals = [1, twin.rotation_galois(1, ch.n)]
        seeds = rng.integers(0, 2**32, (2, 8), dtype=np.uint64).astype(np.uint32)
        err = rng.integers(-3, 4, (2, ch.dnum, ch.n)).astype(np.int64)
        keys = pa.Keys(ctx, gals, seeds=seeds, secret=s, errors=err, bits=0)
        _SETUP[name] = (ch, ctx, keys)
    return _SETUP[name]


def both(ctx, fn):
    """fn() run with every streamed conversion on, then off; the context's setting restored"""
    prev = ctx.conv_fusion(7)
    try:
        a = fn()
        ctx.conv_fusion(0)
        b = fn()
    finally:
        ctx.conv_fusion(prev)
    return a, b


@pytest.mark.parametrize("name,tops", [("c5", [46, 31, 16, 0]), ("c3", [29, 20, 9]), ("t12", [19, 8, 2]),
                                       ("t14", [25, 15])])
def test_rotation_fused_equals_unfused(stream, name, tops):
    ch, ctx, keys = setup(name)
    rng = np.random.default_rng(11)
    for top in tops:
        say(f"[conv_cols] {name} N=2^{ch.logn} kp={len(ch.p)} top={top}: rotation, fused vs bconv + ntt_fwd")
        x = pa.DevBuf.from_array(random_ct(ch, top, rng)[0])
        out = ctx.ct_buf()

        def run():
            out.zero()
            ctx.rotate(keys, 1, x, top, out, stream)
            stream.sync()
            return out.download((2, ch.rows, ch.n))

        a, b = both(ctx, run)
        assert (a[:, : top + 1] == b[:, : top + 1]).all()


@pytest.mark.parametrize("name,tops", [("c5", [46, 33, 17, 2]), ("c3", [29, 12, 2]), ("t12", [19, 5])])
def test_product_rescale_fused_equals_unfused(stream, name, tops):
    """the relinearized product and its two-prime rescale in one ModDown (the exact conversion of kp + 2 sources),
    K = 1 and K = 2 pairs"""
    ch, ctx, keys = setup(name)
    rng = np.random.default_rng(12)
    for top in tops:
        for K in (1, 2):
            say(f"[conv_cols] {name} top={top} K={K}: product + rescale, fused vs bconv + ntt_fwd")
            a = pa.DevBuf.from_array(random_ct(ch, top, rng, K))
            b = pa.DevBuf.from_array(random_ct(ch, top, rng, K))
            out = ctx.ct_buf(K)

            def run():
                out.zero()
                ctx.mul_relin_rescale(keys, a, b, top, out, stream, K=K)
                stream.sync()
                return out.download((K, 2, ch.rows, ch.n))

            x, y = both(ctx, run)
            assert (x[:, :, : top - 1] == y[:, :, : top - 1]).all()


def test_modup_digits_fused_equal_unfused(stream):
    """the ModUp alone: every digit's rows of the workspace, C5 at a top inside the third digit"""
    ch, ctx, keys = setup("c5")
    rng = np.random.default_rng(13)
    top = 40
    x = pa.DevBuf.from_array(random_ct(ch, top, rng)[0])
    say(f"[conv_cols] c5 top={top}: ModUp digits, fused vs bconv + ntt_fwd")

    def run():
        ctx.modup(x, top, stream)
        stream.sync()
        return ctx.modup_digits(stream)

    a, b = both(ctx, run)
    assert a.shape == b.shape
    for d in range(ch.dnum):
        own = set(range(d * ch.alpha, min((d + 1) * ch.alpha, top + 1)))
        if not own:
            continue
        tgt = [t for t in range(top + 1) if t not in own] + [len(ch.q) + k for k in range(len(ch.p))]
        assert (a[d, tgt] == b[d, tgt]).all(), d
    assert ctx.conv_fusion() == 3
