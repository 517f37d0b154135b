"""The full-slot bootstrap at its workload shape, N = 2^16 with 2^15 complex slots: ModRaise of a 1-limb ciphertext to
47 limbs, CoeffToSlot (4 BSGS levels), EvalMod on the real and imaginary parts (two lanes, as the benchmark runs it),
SlotToCoeff (3 levels), every level's babies in the extended basis (one ModDown per giant step), 13 limbs out, on the
chain of 47 Q + 16 special 30-bit primes with dnum 3 and 80 rotation keys plus the relinearization key.

Every output residue of the GPU composite equals the same composite run on the oracle's operations (tests/bts_ops.py)
with the same keys, word for word; the output decrypts to the input's message within 2^-16, and to the plaintext slots
(uniform in [-1, 1] + i [-1, 1], encoded at scale 2^25 with a Gaussian error of sigma 3.19) at 11.65 bits or better:
the precision the reference prints for its plain StC-first bootstrap, bits = log2(max |X| / max error)
(crates/pc-tools/src/bts_stc_first.rs:1364). The oracle's run takes about a minute on 16 host threads.
"""
import math
import os
import sys
import time

import numpy as np
import pytest

import perseus_amd as pa
from perseus_amd import bootstrap as B
from perseus_amd.encoding import decode, encode
from tests import twin
from tests.bts_ops import OracleOps
from tests.test_bootstrap import decrypt_slots, setup_oracle
from tests.test_oracle_ks import encrypt

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.timeout(1200)
def test_bootstrap_c5_matches_the_oracle():
    say("[bootstrap c5] N=2^16, 2^15 slots, 47 Q + 16 special primes, dnum 3, 1 -> 13 limbs, the two EvalMod chains "
        "batched (K = 2): oracle keys")
    twin.set_threads(min(16, os.cpu_count() or 1))
    ch = pa.preset("c5")
    t0 = time.time()
    S = setup_oracle(logn=ch.logn, seed=55, fused=True, chain=(ch.q, ch.p, ch.dnum))
    par = S["par"]
    say(f"[bootstrap c5] {len(S['gal'])} rotation keys from the oracle in {time.time() - t0:.1f} s")
    rng = np.random.default_rng(505)
    z = rng.uniform(-1, 1, par.n) + 1j * rng.uniform(-1, 1, par.n)
    m = np.rint(encode(z, par.N, par.delta_in)).astype(np.int64)
    ct, me = encrypt(S["oc"], S["s_eval"], m, rng, 0)
    # the GPU composite: the oracle's keys uploaded, the relinearization key generated on the device from the same
    # secret, seed and errors (device key generation equals the oracle's, tests/test_gpu_parity.py)
    ctx = pa.Context(ch, k_rot=8, k_max=8)
    keys = pa.Keys(ctx, S["gal"], seeds=S["seeds"], b=S["bs"])
    relin = pa.Keys(ctx, [1], seeds=S["rseed"][None], secret=S["s"], errors=np.stack(S["errs"])[None], relin=True)
    st = pa.Stream()
    ops = B.GpuOps(ctx, keys, relin, S["levels"], S["conj"], st)
    boot = B.Bootstrap(ops, par, ch.q, special=ch.p, fuse_stc=True)
    assert boot.pair
    boot.prepare()
    x = pa.DevBuf.from_array(ct)
    say("[bootstrap c5] GPU run")
    out = boot.run(B.View(x))
    st.sync()
    got = out.h.buf.download((2, ctx.rows, ctx.n), offset=out.h.off, words=ctx.ct_words)
    say(f"[bootstrap c5] GPU output at top {out.top}, scale 2^{math.log2(out.scale):.2f}; oracle run")
    del boot, ops, keys, relin, ctx
    t0 = time.time()
    S["boot"].prepare()
    want = S["boot"].run((ct[None], 0))
    say(f"[bootstrap c5] oracle composite in {time.time() - t0:.1f} s")
    assert out.top == want.top == 12 and out.scale == want.scale
    wh = OracleOps.get(want.h)
    for part in range(2):
        for t in range(out.top + 1):
            assert (got[part, t] == wh[part, t]).all(), f"part {part} limb {t} differs from the oracle"
    slots = decrypt_slots(S, got, out.top, out.scale)
    ref = decode(me.astype(np.float64), par.N, par.delta_in)  # the input's message, its encryption error included
    err_in = float(np.abs(slots - ref).max())
    e_pl = max(float(np.abs(slots.real - z.real).max()), float(np.abs(slots.imag - z.imag).max()))
    amp = max(float(np.abs(z.real).max()), float(np.abs(z.imag).max()))
    bits = math.log2(amp / e_pl)
    say(f"[bootstrap c5] max |error| vs the input's message {err_in:.3g}; vs the plaintext {e_pl:.3g} "
        f"({bits:.2f} bits)")
    assert err_in < 2.0 ** -16
    assert bits >= 11.65
