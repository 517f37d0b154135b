"""Banded switching keys (crates/pc-gpu/src/keys.rs:81-103 KskShape::banded, :351-376 KeySetSpec::with_band): a key
group that stores, per key, only the digits whose first prime id is <= q_top and in each the Q rows 0..=q_top plus the
special rows (pcx_keys_new_banded). Its rotations at any top <= q_top equal the oracle's with the full key, word for
word, at the C3 shape (31-bit primes; dense b and b packed at 31 bits) and the C5 shape (30-bit primes, packed at 30
bits): single rotations, hoisted batches and summed rotations (KS_SUM); a ciphertext above the band is refused; the
stored rows download as the band of the full key; a bundle entry of a banded shape loads through wire.load_keys."""
import io
import sys

import numpy as np
import pytest

import perseus_amd as pa
from perseus_amd import wire
from perseus_amd.engine import band_digits, band_rows
from tests import twin

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def stream():
    assert pa.device_count() >= 1, "no GPU visible"
    return pa.Stream()


_CTX = {}


def setup(name, steps, seed):
    key = (name, tuple(steps), seed)
    if key not in _CTX:
        ch = pa.preset(name)
        ctx = pa.Context(ch, k_rot=4)
        oc = twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum)
        g = twin.Prng([seed, 3, 1, 4, 1, 5, 9, 2], 0)
        s_eval = oc.secret_eval(g.sparse_ternary(ch.n, 192))
        gals = [twin.rotation_galois(r, ch.n) for r in steps]
        ks = [oc.rotation_key(g, s_eval, x) for x in gals]
        _CTX[key] = (ch, ctx, oc, gals, np.stack([k[0] for k in ks]), [k[1] for k in ks])
    return _CTX[key]


def random_ct(ch, top, seed):
    rng = np.random.default_rng(seed)
    ct = np.zeros((2, ch.rows, ch.n), np.uint32)
    for part in range(2):
        for t in range(top + 1):
            ct[part, t] = rng.integers(0, ch.primes[t], ch.n)
    return ct


@pytest.mark.parametrize("name,q_top,tops,bits", [("c3", 19, [19, 12, 3], 0), ("c3", 9, [9, 0], 31),
                                                  ("c5", 20, [20, 7], 30), ("c5", 31, [31], 0)])
def test_banded_rotations_equal_the_full_keys(stream, name, q_top, tops, bits):
    steps = [1, 2, 5, 64]
    ch, ctx, oc, gals, seeds, bs = setup(name, steps, 17)
    say(f"[banded] {name} q_top={q_top} tops={tops} bits={bits}: {band_digits(ctx, q_top)} of {ch.dnum} digits")
    banded = [band_rows(b, ctx, q_top) for b in bs]
    assert banded[0].shape == (band_digits(ctx, q_top), q_top + 1 + len(ch.p), ch.n)
    keys = pa.Keys(ctx, gals, seeds=seeds, b=banded, bits=bits, q_top=q_top)
    assert keys.q_top() == q_top and keys.patch_bytes() == 0
    assert (keys.download_b(2) == banded[2]).all()
    for top in tops:
        ct = random_ct(ch, top, top + q_top)
        x = pa.DevBuf.from_array(ct)
        out = ctx.ct_buf(len(steps))
        say(f"[banded] {name} top={top}: rotate, hoisted, sum")
        ctx.rotate(keys, 1, x, top, out, stream)
        stream.sync()
        got = out.download((len(steps), 2, ch.rows, ch.n))[0]
        want = oc.rotate(ct, top, seeds[1], bs[1], gals[1])
        assert (got[:, : top + 1] == want[:, : top + 1]).all(), "rotate"
        ctx.rotate_hoisted(keys, [0, 1, 2, 3], x, top, out, stream)
        stream.sync()
        got = out.download((len(steps), 2, ch.rows, ch.n))
        want = oc.rotate_hoisted(ct, top, seeds, bs, gals)
        for j in range(len(steps)):
            assert (got[j, :, : top + 1] == want[j][:, : top + 1]).all(), f"hoisted {j}"
        one = ctx.ct_buf(1)
        ctx.rotate_sum(keys, [0, 2, 3], x, top, one, stream)
        stream.sync()
        got = one.download((2, ch.rows, ch.n))
        want = oc.rotate_sum(ct, top, seeds[[0, 2, 3]], [bs[0], bs[2], bs[3]], [gals[0], gals[2], gals[3]])
        assert (got[:, : top + 1] == want[:, : top + 1]).all(), "rotate_sum"
    say(f"[banded] {name}: a ciphertext at top {q_top + 1} is refused")
    with pytest.raises(pa.HipError):
        ctx.rotate(keys, 0, ctx.ct_buf(1), q_top + 1, ctx.ct_buf(1), stream)


def test_banded_bundle_entry_loads(stream):
    ch, ctx, oc, gals, seeds, bs = setup("c3", [1, 2, 5, 64], 17)
    q_top, bits = 14, 31
    say(f"[banded] c3: a bundle of two keys banded at {q_top} (packed at {bits} bits) -> load_keys -> rotate")
    rw = wire.packed_row_words(ch.n, bits)
    shape = {"q_top": q_top, "ndig": band_digits(ctx, q_top), "nq": len(ch.q), "kp": len(ch.p)}
    pick = [0, 3]
    entries = [wire.ksk_entry("rot", shape, seeds[r], rw, step=s, galois=gals[r]) for r, s in zip(pick, [1, 64])]
    h = {"chain": ch.name, "params_hash": "t", "contract": "t", "n": ch.n, "bits": bits, "row_words": rw,
         "entries": entries}
    f = io.BytesIO()
    bw = wire.BundleWriter(f, h)
    for r in pick:
        bw.put(wire.pack_ksk(band_rows(bs[r], ctx, q_top), bits, rw))
    bw.finish()
    group, idx = wire.load_keys(wire.BundleReader(io.BytesIO(f.getvalue())), ctx)
    assert idx == [0, 1] and group.q_top() == q_top
    top = 11
    ct = random_ct(ch, top, 5)
    x, out = pa.DevBuf.from_array(ct), ctx.ct_buf(1)
    for j, r in enumerate(pick):
        ctx.rotate(group, j, x, top, out, stream)
        stream.sync()
        want = oc.rotate(ct, top, seeds[r], bs[r], gals[r])
        assert (out.download((2, ch.rows, ch.n))[:, : top + 1] == want[:, : top + 1]).all(), r
    # a shape that does not fit: the digit count of another band
    bad = dict(shape, ndig=ch.dnum)
    h2 = dict(h, entries=[wire.ksk_entry("rot", bad, seeds[0], rw, step=1, galois=gals[0])])
    f2 = io.BytesIO()
    bw = wire.BundleWriter(f2, h2)
    bw.put(wire.pack_ksk(np.concatenate([band_rows(bs[0], ctx, q_top)] * 2)[: ch.dnum], bits, rw))
    bw.finish()
    with pytest.raises(wire.WireError):
        wire.load_keys(wire.BundleReader(io.BytesIO(f2.getvalue())), ctx)
