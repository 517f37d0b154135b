"""The host sampler of key generation (perseus_amd/csrc/drbg.cpp through pcx_drbg_*) against the oracle's samplers,
which are pinned to raw RFC 8439 ChaCha20 words and the reference's draw rules (tests/test_oracle_samplers.py): the
DRBG's words across block and counter boundaries, several keys and streams; the sparse ternary secret; the discrete
Gaussian; and pcx_keygen_draw's seeds and errors against or_rotation_key's draw order. No GPU: the sampler runs on the
host."""
import numpy as np
import pytest

import perseus_amd as pa
from tests import twin


@pytest.mark.parametrize("stream", [0, 1, 7, 0xFFFFFFFF])
def test_drbg_words_equal_the_oracle(stream):
    key = [0x01234567, 0x89ABCDEF, 3, 4, 5, 6, 7, 0xFFFFFFFF]
    a, b = pa.Drbg(key, stream), twin.Prng(key, stream)
    assert [a.u32() for _ in range(100)] == [b.u32() for _ in range(100)]
    assert (a.ksk_seed() == b.ksk_seed()).all()


@pytest.mark.parametrize("n,h", [(1 << 10, 64), (1 << 12, 192), (64, 64), (16, 0)])
def test_sparse_ternary_equals_the_oracle(n, h):
    key = [9, 8, 7, 6, 5, 4, 3, n]
    x = pa.Drbg(key, 3).sparse_ternary(n, h)
    assert (x == twin.Prng(key, 3).sparse_ternary(n, h)).all()
    assert int(np.abs(x).sum()) == h
    with pytest.raises(ValueError):
        pa.Drbg(key, 3).sparse_ternary(n, n + 1)


@pytest.mark.parametrize("sigma", [3.19, 1.0, 10.5])
def test_gaussian_equals_the_oracle(sigma):
    key = [1, 1, 2, 3, 5, 8, 13, 21]
    a = pa.Drbg(key, 2)
    b = twin.Prng(key, 2)
    x = a.gaussian(1 << 14, sigma)
    assert (x == b.gaussian(1 << 14, sigma)).all()
    assert abs(float(np.std(x)) - sigma) < 0.05 * sigma
    # the streams stay aligned after the variable-length draws
    assert a.u32() == b.u32()


def test_keygen_draw_follows_the_rotation_keys_order():
    """seeds and errors of pcx_keygen_draw equal the oracle's rotation key draws: the key's seed (8 words), the error
    streams' key (8 more), then digit d's Gaussian draws from the stream (that key, d); a second key continues the same
    DRBG"""
    n, ndig = 1 << 10, 3
    key = [4, 3, 2, 1, 0, 1, 2, 3]
    seeds, errors = pa.Drbg(key, 9).keygen_draw(2, ndig, n)
    g = twin.Prng(key, 9)
    for r in range(2):
        assert (seeds[r] == g.ksk_seed()).all(), r
        sub = g.ksk_seed()
        for d in range(ndig):
            assert (errors[r, d] == twin.Prng(sub, d).gaussian(n, 3.19)).all(), (r, d)
