"""The SPRU floating-point table entries on the GPU (perseus_amd/csrc/spru.hip) against the oracle, bit for bit:
spru_fft_pass at N = 2^12 (every pass of a whole transform, in sequence) and N = 2^16 (first, middle and last
passes), spru_scatter into 1 and several limbs with ties and negative coefficients, and the launchers' refusals.
"""
import sys

import numpy as np
import pytest

import perseus_amd as pa
from perseus_amd import abi
from perseus_amd._lib import LIB
from tests import twin
from tests.test_oracle_spru import tw_table, zt_table

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def stream():
    assert pa.device_count() >= 1, "no GPU visible"
    return pa.Stream()


def dev(x):
    return pa.DevBuf.from_array(np.ascontiguousarray(x, np.complex128).view(np.uint32))


def get(buf, shape):
    return buf.download((int(np.prod(shape)) * 4,)).view(np.complex128).reshape(shape)


def fft_pass(stream, bin_, bout, btw, ns, batch, logn):
    a = abi.SpruFftArgs()
    a.inp, a.out, a.tw, a.ns, a.batch = bin_.ptr.value, bout.ptr.value, btw.ptr.value, ns, batch
    rc = abi.call("spru_fft_pass", a, stream, logn)
    assert rc == 0, rc
    stream.sync()


@pytest.mark.parametrize("logn,passes", [(12, None), (16, [1, 64, 1 << 15])])
def test_fft_pass(stream, logn, passes):
    n, batch = 1 << logn, 3
    say(f"[spru_fft_pass] logn={logn} passes={passes or 'all'}")
    rng = np.random.default_rng(logn)
    x = rng.normal(size=(batch, n)) * 1e4 + 1j * rng.normal(size=(batch, n))
    tw = tw_table(n)
    btw = dev(tw)
    if passes is None:
        bx, by = dev(x), dev(np.zeros_like(x))
        y, ns = x, 1
        while ns < n:
            fft_pass(stream, bx, by, btw, ns, batch, logn)
            y = twin.spru_fft_pass(y, tw, ns)
            assert (get(by, (batch, n)).view(np.uint64) == y.view(np.uint64)).all(), ns
            bx, by = by, bx
            ns *= 2
        assert np.abs(y - np.fft.fft(x, axis=-1)).max() < 1e-12 * n * 1e4
    else:
        bx, by = dev(x), dev(np.zeros_like(x))
        for ns in passes:
            fft_pass(stream, bx, by, btw, ns, batch, logn)
            want = twin.spru_fft_pass(x, tw, ns)
            assert (get(by, (batch, n)).view(np.uint64) == want.view(np.uint64)).all(), ns


@pytest.mark.parametrize("logn,nl,scale", [(12, 1, 1.0), (16, 5, 2.0 ** 30)])
def test_scatter(stream, logn, nl, scale):
    n, batch = 1 << logn, 2
    say(f"[spru_scatter] logn={logn} nl={nl}")
    ch = pa.preset("small31" if logn == 12 else "c3")
    ctx = pa.Context(ch, k_rot=1)
    primes = [int(p) for p in ch.primes[:nl]]
    rng = np.random.default_rng(nl)
    y = (rng.normal(size=(batch, n)) + 1j * rng.normal(size=(batch, n))) * n * 1e6 / scale
    zt = zt_table(n)
    zt[:6] = 1.0
    y[0, :6] = np.array([2.5, 3.5, -2.5, -3.5, 0.5, -0.5]) * n / scale + 5j
    y[1, 0] = -(2.0 ** 61) * n / scale
    stride = nl * n + 256
    out = pa.DevBuf(batch * stride)
    by, bz = dev(y), dev(zt)
    a = abi.SpruScatterArgs()
    a.y, a.out, a.zt, a.pr = by.ptr.value, out.ptr.value, bz.ptr.value, LIB.pcx_ctx_primes(ctx.h)
    a.scale, a.nl, a.batch, a.out_stride = scale, nl, batch, stride
    rc = abi.call("spru_scatter", a, stream, logn)
    assert rc == 0, rc
    stream.sync()
    got = out.download((batch, stride))[:, : nl * n].reshape(batch, nl, n)
    want = twin.spru_scatter(y, zt, primes, scale)
    assert (got == want).all()
    assert [int(got[0, 0, k]) for k in range(4)] == [2, 4, primes[0] - 2, primes[0] - 4]


def test_refusals(stream):
    n = 1 << 12
    b = pa.DevBuf(4 * n)
    t = pa.DevBuf(2 * n)
    a = abi.SpruFftArgs()
    for ns, same in ((3, False), (0, False), (n, False), (n // 2, True)):
        a.inp, a.out, a.tw, a.ns, a.batch = b.ptr.value, (b if same else t).ptr.value, t.ptr.value, ns, 1
        assert abi.call("spru_fft_pass", a, stream, 12) == -1, (ns, same)
    s = abi.SpruScatterArgs()
    s.y, s.out, s.zt, s.pr, s.nl, s.batch = b.ptr.value, t.ptr.value, b.ptr.value, b.ptr.value, 0, 1
    assert abi.call("spru_scatter", s, stream, 12) == -1
