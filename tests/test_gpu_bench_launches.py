"""The launches bench.py times, checked against the oracle as they run there:
- the C3 hoisted batch (N = 2^16, 30 limbs of 31-bit primes, dnum 3, 6 special primes) over every step of the bench's
  step set ({1..16} and 32..2^15: 26 key switches and the identity) on a context of k_rot 26, keys generated on the
  device from a ternary secret, Gaussian errors and ChaCha seeds as the bench makes them: the headline's dense keys
  (the fused dot with the key group's retry-value table, dot_fast<3, true, 4, 0, false>) and the drop-in path's PackedSeeded
  keys at 31 bits through the kernel table alone; every one of the 27 outputs word for word against the oracle's
  hoisted rotations with the same keys (their b downloaded);
- the C4 attention scoring as one batch of six ciphertexts (attention.score_batch: pcx_mul_plain_k, pcx_rescale_k and
  pcx_rotate_and_sum_k at K = 6 on a k_max = k_rot = 6 context): each ciphertext's scores word for word against the
  oracle's composition (plaintext product, two-prime rescale, the radix-8 ladder)."""
import os
import sys

import numpy as np
import pytest

import bench
import perseus_amd as pa
from oracle import em
from perseus_amd import attention
from perseus_amd.bootstrap import View
from tests import twin

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def stream():
    assert pa.device_count() >= 1, "no GPU visible"
    twin.set_threads(min(16, os.cpu_count() or 1))
    return pa.Stream()


def bench_keys_material(n, gals, dnum, seed, stream):
    """the bench's key material (bench.py main): the weight-192 ternary secret and each key's seed and Gaussian errors
    from the bench's DRBG streams (bench.draw_secret, bench.key_draws: the reference's samplers and keygen order)"""
    rng = np.random.default_rng(seed)
    secret = bench.draw_secret(pa, n)
    seeds, errors = bench.key_draws(pa, stream, len(gals), dnum, n)
    return secret, seeds, errors, rng


@pytest.mark.timeout(600)
@pytest.mark.parametrize("layout", ["dense", "packed31_table"])
def test_c3_hoisted_batch_of_the_bench(stream, layout):
    ch = pa.preset("c3")
    n, top = ch.n, len(ch.q) - 1
    gals = [pow(5, s % (n // 2), 2 * n) for s in bench.STEPS_SET]
    R = sum(1 for g in gals if g != 1)
    assert R == 26 and len(gals) == 27
    say(f"[bench launches] c3 hoisted batch, {R} key switches + the identity, keys {layout}")
    secret, seeds, errors, rng = bench_keys_material(n, gals, ch.dnum, 2024, 1)
    ctx = pa.Context(ch, k_rot=R)
    bits = 0
    if layout != "dense":
        ctx.table_only(True)
        bits = 31
    keys = pa.Keys(ctx, gals, seeds=seeds, bits=bits, secret=secret, errors=errors)
    assert (keys.patch_bytes() > 0) == (layout == "dense")
    ct = np.zeros((2, ch.rows, n), np.uint32)
    for part in range(2):
        for t in range(top + 1):
            ct[part, t] = rng.integers(0, ch.primes[t], n)
    dev, outs = pa.DevBuf.from_array(ct), ctx.ct_buf(len(gals))
    ctx.rotate_hoisted(keys, list(range(len(gals))), dev, top, outs, stream)
    stream.sync()
    got = outs.download((len(gals), 2, ch.rows, n))
    say("[bench launches] the oracle's hoisted batch with the downloaded keys")
    oc = twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum)
    bs = [keys.download_b(i) for i in range(len(gals))]
    want = oc.rotate_hoisted(ct, top, seeds, bs, gals)
    for j in range(len(gals)):
        assert (got[j, :, : top + 1] == want[j][:, : top + 1]).all(), f"step {bench.STEPS_SET[j]}"


@pytest.mark.timeout(600)
def test_c4_score_batch_of_the_bench(stream):
    ch = pa.preset("c4")
    n, top = ch.n, len(ch.q) - 1
    nc = attention.n_cts()
    steps = attention.ladder_steps()
    gals = [pow(5, r, 2 * n) for r in steps]
    say(f"[bench launches] c4 score_batch: {nc} ciphertexts, ladder radix 2^{attention.RADIX_BITS}, "
        f"{len(gals)} keys")
    secret, seeds, errors, rng = bench_keys_material(n, gals, ch.dnum, 404, 4)
    ctx = pa.Context(ch, k_rot=nc, k_max=nc)
    keys = pa.Keys(ctx, gals, seeds=seeds, secret=secret, errors=errors)
    cts = np.zeros((nc, 2, ch.rows, n), np.uint32)
    for c in range(nc):
        for part in range(2):
            for t in range(top + 1):
                cts[c, part, t] = rng.integers(0, ch.primes[t], n)
    pts = np.zeros((nc, ch.rows, n), np.uint32)
    for c in range(nc):
        for t in range(top + 1):
            pts[c, t] = rng.integers(0, ch.primes[t], n)
    xb, ob, tb = pa.DevBuf.from_array(cts), ctx.ct_buf(nc), ctx.ct_buf(nc)
    pbs = [pa.DevBuf.from_array(p) for p in pts]
    attention.score_batch(ctx, keys, View(xb), pbs, top, View(ob), View(tb), stream)
    stream.sync()
    got = ob.download((nc, 2, ch.rows, n))
    oc = twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum)
    bs = [keys.download_b(i) for i in range(len(gals))]
    for c in range(nc):
        say(f"[bench launches] c4 ciphertext {c}: the oracle's composition")
        prod = oc.ct_zeros()
        prod[:, : top + 1] = em.mul_add_n(ch.primes, [(cts[c][None, :, : top + 1], pts[c])])[0]
        rs = oc.rescale(prod, top, 2)
        want = oc.rotate_and_sum(rs, top - 2, 1, attention.BLOCK, seeds, bs, gals, attention.RADIX_BITS)
        assert (got[c][:, : top - 1] == want[:, : top - 1]).all(), c
