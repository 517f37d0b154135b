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


# ----------------------------------------------------------------------------------------------- import / export
META = {"level": 0, "deg": 1, "nf": 2.0 ** 30, "slots": 2048, "tag": None}


def _bytes(h, data):
    f = io.BytesIO()
    wire.write_ct(f, h, data)
    return f.getvalue()


def test_import_coefficient_form_frames():
    say("[wire] small chain: import_ct of a short-c0 DRBG-seeded frame and a subring frame (forward NTT on the device)")
    ch = pa.preset("small")
    ctx, oc = pa.Context(ch, k_rot=1), twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum)
    st = pa.Stream()
    n, rows = ch.n, 3
    q = ch.q[:rows]
    rng = np.random.default_rng(21)
    # short c0: coefficient rows rounded to their top bits, seeds for c1 (DRBG)
    coef = np.stack([rng.integers(0, p, n) for p in q]).astype(np.uint32)
    seeds = rng.integers(0, 1 << 32, (rows, 8), dtype=np.uint64).astype(np.uint32)
    w, bits = wire.pack_dropped(q, coef, 12)
    h = wire.ct_header("t", n, 1, rows, META, seeded=True, drop=12, bits=bits, sparse=True)
    raw = _bytes(h, np.concatenate([w, seeds.reshape(-1)]))
    with pytest.raises(wire.WireError, match="client"):
        wire.import_ct(ctx, raw, st)  # as the reference's import_ct: a short-c0 frame is expanded first
    buf, hh = wire.import_ct(ctx, wire.expand_frame(raw, ch.q), st)
    assert hh.get("sparse") and hh.get("coeff0")
    got = buf.download((2, ch.rows, n))
    want0 = oc.ntt_fwd(wire.unpack_dropped(q, w, 12, n), list(range(rows)))
    assert (got[0, :rows] == want0).all()
    for r in range(rows):
        assert (got[1, r] == wire.drbg_row(seeds[r], q[r], n)).all()
    # a subring client's frame: both parts in coefficient form over N/2 coefficients, lifted X -> X^2, then NTT'd
    hs = wire.ct_header("t", n // 2, 1, rows, dict(META, slots=n // 4), coeff0=True, coeff1=True)
    small = np.stack([np.stack([rng.integers(0, p, n // 2) for p in q]) for _ in range(2)]).astype(np.uint32)
    buf, hh = wire.import_ct(ctx, _bytes(hs, small), st)
    got = buf.download((2, ch.rows, n))
    big = np.zeros((2, rows, n), np.uint32)
    big[:, :, ::2] = small
    for part in range(2):
        assert (got[part, :rows] == oc.ntt_fwd(big[part], list(range(rows)))).all(), part
    assert hh["n"] == n
    # a compressed frame is a client's to decrypt
    hc = wire.ct_header("t", n, 1, 2, META, bits=20)
    with pytest.raises(wire.WireError, match="client"):
        wire.import_ct(ctx, _bytes(hc, np.zeros(wire.ct_words(hc), np.uint32)), st)


def test_export_full_and_compressed():
    say("[wire] small chain: export_ct full and compressed (inverse NTT on the device, rounded CRT at 24 bits)")
    ch = pa.preset("small")
    ctx, oc = pa.Context(ch, k_rot=1), twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum)
    st = pa.Stream()
    n, top = ch.n, 1
    rng = np.random.default_rng(22)
    ct = np.zeros((2, ch.rows, n), np.uint32)
    for part in range(2):
        for t in range(top + 1):
            ct[part, t] = rng.integers(0, ch.q[t], n)
    buf = pa.DevBuf.from_array(ct)
    h, d = wire.read_ct(io.BytesIO(wire.export_ct(ctx, buf, top, META, "t", st)))
    assert (d.reshape(2, top + 1, n) == ct[:, : top + 1]).all()
    h, d = wire.read_ct(io.BytesIO(wire.export_ct(ctx, buf, top, META, "t", st, bits=24)))
    assert h["bits"] == 24 and (buf.download((2, ch.rows, n)) == ct).all(), "the source is unchanged"
    q = ch.q[: top + 1]
    pw = wire.packed_words(n, 24)
    for part in range(2):
        coef = oc.ntt_inv(ct[part, : top + 1].copy(), list(range(top + 1)))
        assert (d[part * pw:(part + 1) * pw] == wire.pack_frame_part(q, coef, 24)).all(), part
