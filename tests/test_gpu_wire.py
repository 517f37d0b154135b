"""Keys from a reference-format bundle (perseus_amd.wire) drive the engine: oracle rotation keys written into a bundle
(b bit-packed at 30 bits, the seeds in the header), read back and loaded into a key group, rotate a ciphertext on the
GPU to the oracle's words, and a regenerable ciphertext frame expands into the ciphertext that is rotated. Each test
prints its case before the GPU runs.
"""
import io
import sys

import numpy as np
import pytest

import perseus_amd as pa
from perseus_amd import wire
from tests import twin

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_bundle_keys_rotate_like_the_oracle():
    say("[wire] small chain: bundle keys (bits 30) -> key group -> rotations vs the oracle")
    assert pa.device_count() >= 1, "no GPU visible"
    ch = pa.preset("small")
    ctx, oc = pa.Context(ch, k_rot=2), twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum)
    n, top = ch.n, len(ch.q) - 1
    g = twin.Prng([9, 9, 1, 2, 3, 4, 5, 6], 0)
    s_eval = oc.secret_eval(g.sparse_ternary(n, 64))
    steps = [1, 5]
    gals = [twin.rotation_galois(r, n) for r in steps]
    keys = [oc.rotation_key(g, s_eval, x) for x in gals]
    bits = 30
    rw = wire.packed_row_words(n, bits)
    shape = {"q_top": top, "ndig": ch.dnum, "nq": len(ch.q), "kp": len(ch.p)}
    entries = [wire.ksk_entry("rot", shape, k[0], rw, step=r, galois=x) for r, x, k in zip(steps, gals, keys)]
    h = {"chain": ch.name, "params_hash": "t", "contract": "t", "n": n, "bits": bits, "row_words": rw,
         "entries": entries}
    f = io.BytesIO()
    bw = wire.BundleWriter(f, h)
    for k in keys:
        bw.put(wire.pack_ksk(k[1], bits, rw))
    bw.finish()
    group, idx = wire.load_keys(wire.BundleReader(io.BytesIO(f.getvalue())), ctx)
    assert idx == [0, 1]
    # the input as a regenerable ciphertext frame (c0 rows and c1 seeds)
    rng = np.random.default_rng(4)
    c0 = np.stack([rng.integers(0, p, n) for p in ch.q]).astype(np.uint32)
    seeds = rng.integers(0, 1 << 32, (len(ch.q), 8), dtype=np.uint64).astype(np.uint32)
    hc = {"params_hash": "t", "n": n, "k": 1, "rows": len(ch.q), "seeded": True, "regen": True,
          "meta": {"level": 0, "deg": 1, "nf": 2.0 ** 30, "slots": n // 2, "tag": None}}
    fc = io.BytesIO()
    wire.write_ct(fc, hc, np.concatenate([c0.reshape(-1), seeds.reshape(-1)]))
    hh, d = wire.read_ct(io.BytesIO(fc.getvalue()))
    ct = np.zeros((2, ch.rows, n), np.uint32)
    ct[:, : top + 1] = wire.expand_ct(hh, d, ch.q)[0]
    st = pa.Stream()
    x, out = pa.DevBuf.from_array(ct), ctx.ct_buf(1)
    for r, (seed, b) in enumerate(keys):
        ctx.rotate(group, r, x, top, out, st)
        st.sync()
        got = out.download((2, ch.rows, n))
        want = oc.rotate(ct, top, seed, b, gals[r])
        assert (got[:, : top + 1] == want[:, : top + 1]).all(), r
