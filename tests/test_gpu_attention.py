"""Encrypted attention scoring on the GPU at the C4 shape (12 heads x 64, 512 tokens, N = 2^16, complex packing at
scale 2^40): the keys encrypted under a ternary secret (h = 192), the query a plaintext at the scale of the two primes
the rescale drops, per ciphertext mul_plain -> rescale -> rotate-and-sum over the 64-slot head blocks. The decrypted
scores must match the float64 plaintext scores, and the first ciphertext's words must equal the oracle's composition
of the same steps (plaintext product, rescale, ladder) word for word.
"""
import sys

import numpy as np
import pytest

import perseus_amd as pa
from oracle import em
from perseus_amd import attention, encoding
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


def setup(ch, ctx, oc, seed=2025, radix_bits=attention.RADIX_BITS):
    n, top = ch.n, len(ch.q) - 1
    g = twin.Prng([seed, 1, 2, 3, 4, 5, 6, 7], 0)
    s = g.sparse_ternary(n, 192)
    s_eval = oc.secret_eval(s)
    gals = [twin.rotation_galois(r, n) for r in attention.ladder_steps(radix_bits)]
    seeds = np.stack([g.ksk_seed() for _ in gals])
    errs = np.stack([np.stack([g.gaussian(n) for _ in range(ch.dnum)]) for _ in gals])
    keys = pa.Keys(ctx, gals, seeds=seeds, secret=s, errors=errs)
    rng = np.random.default_rng(seed)
    K = rng.normal(size=(attention.TOKENS, attention.HEADS * attention.HEAD_DIM))
    q = rng.normal(size=(attention.HEADS, attention.HEAD_DIM))
    delta = 2.0 ** 40
    cts = []
    for z in attention.key_slots(K, n):
        m = np.rint(encoding.encode(z, n, delta)).astype(np.int64)
        ct, _ = encrypt(oc, s_eval, m, rng, top)
        cts.append(ct)
    ptscale = float(ch.q[top]) * float(ch.q[top - 1])
    pts = []
    for z in attention.query_slots(q, n):
        rows = encoding.to_residues(encoding.encode(z, n, ptscale), ch.primes[: top + 1])
        full = np.zeros((ch.rows, n), np.uint32)
        full[: top + 1] = oc.ntt_fwd(rows, list(range(top + 1)))
        pts.append(full)
    want = np.einsum("hd,thd->ht", q, K.reshape(attention.TOKENS, attention.HEADS, attention.HEAD_DIM))
    return dict(s_eval=s_eval, gals=gals, seeds=seeds, keys=keys, cts=cts, pts=pts, want=want, delta=delta, top=top)


@pytest.mark.parametrize("radix_bits", [1, 2, 3])
def test_attention_scores_decrypt_and_match_the_oracle(stream, radix_bits):
    say(f"[attention] c4: 6 ciphertexts, mul_plain -> rescale -> rotate_and_sum over 64 slots, radix 2^{radix_bits}")
    ch = pa.preset("c4")
    ctx = pa.Context(ch, k_rot=1)
    oc = twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum)
    S = setup(ch, ctx, oc, radix_bits=radix_bits)
    top, n = S["top"], ch.n
    outs = []
    tmp = ctx.ct_buf(1)
    for ct, pt in zip(S["cts"], S["pts"]):
        bct, bpt, out = pa.DevBuf.from_array(ct), pa.DevBuf.from_array(pt), ctx.ct_buf(1)
        attention.score(ctx, S["keys"], bct, bpt, top, out, tmp, stream, radix_bits)
        stream.sync()
        outs.append(out.download((2, ch.rows, n)))
    zs = []
    for o in outs:
        coef = encoding.from_residues(decrypt(oc, S["s_eval"], o, top - 2), ch.primes[: top - 1])
        zs.append(encoding.decode(coef, n, S["delta"]))
    got = attention.scores_from_slots(zs)
    err = np.abs(got - S["want"]).max()
    say(f"[attention] max |score error| = {err:.3g} (scores up to {np.abs(S['want']).max():.1f})")
    assert err < 1e-3
    # the first ciphertext's words against the oracle's composition
    x = S["cts"][0]
    prod = oc.ct_zeros()
    prod[:, : top + 1] = em.mul_add_n(ch.primes, [(x[None, :, : top + 1], S["pts"][0])])[0]
    rs = oc.rescale(prod, top, 2)
    bs = [S["keys"].download_b(i) for i in range(len(S["gals"]))]
    want0 = oc.rotate_and_sum(rs, top - 2, 1, attention.BLOCK, S["seeds"], bs, S["gals"], radix_bits)
    assert (outs[0][:, : top - 1] == want0[:, : top - 1]).all()


def test_attention_scoring_graph_replays(stream):
    """One ciphertext's scoring captured into a HIP graph and replayed three times, with eager work (the scoring of
    another ciphertext into the same workspace) and a cleared output between replays: every replay equals the eager
    result word for word."""
    say("[attention] c4 scoring graph, 3 replays")
    ch = pa.preset("c4")
    ctx = pa.Context(ch, k_rot=1)
    oc = twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum)
    S = setup(ch, ctx, oc, seed=77)
    top, n = S["top"], ch.n
    bct = [pa.DevBuf.from_array(c) for c in S["cts"][:2]]
    bpt = [pa.DevBuf.from_array(p) for p in S["pts"][:2]]
    eager, other, out, tmp = ctx.ct_buf(1), ctx.ct_buf(1), ctx.ct_buf(1), ctx.ct_buf(1)
    attention.score(ctx, S["keys"], bct[0], bpt[0], top, eager, tmp, stream)
    stream.sync()
    want = eager.download((2, ch.rows, n))
    graph = pa.Graph(stream, lambda: attention.score(ctx, S["keys"], bct[0], bpt[0], top, out, tmp, stream))
    for rep in range(3):
        out.zero()
        attention.score(ctx, S["keys"], bct[1], bpt[1], top, other, tmp, stream)
        stream.sync()
        graph.launch(stream)
        stream.sync()
        got = out.download((2, ch.rows, n))
        assert (got[:, : top - 1] == want[:, : top - 1]).all(), rep
