"""The bootstrap composite on the GPU (perseus_amd.bootstrap.GpuOps) at N = 2^12: word for word equal to the same
composite run on the oracle's operations (tests/bts_ops.py) with the same keys, its decryption equal to the input's
message, and a second run (the buffer pool and the cached constants reused) giving the same words. Each test prints its
case before the GPU runs.
"""
import sys

import numpy as np
import pytest

import perseus_amd as pa
from perseus_amd import bootstrap as B
from tests.bts_ops import OracleOps
from tests.test_bootstrap import decrypt_slots, input_ct, setup_oracle

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def gpu_boot(S, lanes=1):
    """lanes 1: one stream; 2: the imaginary part's EvalMod on a second context and stream; "pair": both EvalMod
    chains batched (K = 2) on a k_max 4 context (giant steps batched too)"""
    par, q, oc = S["par"], S["q"], S["oc"]
    ch = pa.Chain("bts12", par.logn, q, [int(p) for p in oc.primes[len(q):]], oc.dnum)
    ctx = pa.Context(ch, k_rot=8, k_max=4 if lanes == "pair" else 1)
    keys = pa.Keys(ctx, S["gal"], seeds=S["seeds"], b=S["bs"])
    relin = pa.Keys(ctx, [1], seeds=S["rseed"][None], secret=S["s"], errors=np.stack(S["errs"])[None], relin=True)
    st = pa.Stream()
    ops = B.GpuOps(ctx, keys, relin, S["levels"], S["conj"], st)
    ops2 = None
    if lanes == 2:
        ctx2 = pa.Context(ch, k_rot=1)
        relin2 = pa.Keys(ctx2, [1], seeds=S["rseed"][None], secret=S["s"], errors=np.stack(S["errs"])[None],
                         relin=True)
        ops2 = B.GpuOps(ctx2, None, relin2, S["levels"], S["conj"], pa.Stream())
        ops2.keep = (ctx2, relin2)
    boot = B.Bootstrap(ops, par, q, ops2, special=S["p"] if S["fused"] else None, fuse_stc=S["fused"] != "cts")
    assert boot.pair == (lanes == "pair")
    boot.prepare()
    return ctx, keys, relin, st, ops, boot


@pytest.mark.parametrize("lanes,fused", [(1, False), (2, True), (1, True), ("pair", False), ("pair", True),
                                         ("pair", "cts")])
def test_bootstrap_gpu_matches_the_oracle(lanes, fused):
    say(f"[bootstrap] N=2^12, {lanes} EvalMod lane(s), fused babies {fused}: GPU composite vs the oracle composite, "
        "decryption, rerun")
    S = setup_oracle(fused=fused)
    rng = np.random.default_rng(9)
    z, ct, me = input_ct(S, rng)
    ctx, keys, relin, st, ops, boot = gpu_boot(S, lanes)
    say(f"[bootstrap] {len(S['gal'])} keys, top {boot.T} -> {boot.top_out}")
    x = pa.DevBuf.from_array(ct)
    out = boot.run(B.View(x))
    st.sync()
    got = out.h.buf.download((2, ctx.rows, ctx.n), offset=out.h.off, words=ctx.ct_words)
    S["boot"].prepare()
    want = S["boot"].run((ct[None], 0))
    assert out.top == want.top and out.scale == want.scale
    wh = OracleOps.get(want.h)
    assert (got[:, : out.top + 1] == wh[:, : out.top + 1]).all(), "GPU == oracle, word for word"
    from perseus_amd.encoding import decode

    slots = decrypt_slots(S, got, out.top, out.scale)
    ref = decode(me.astype(np.float64), S["par"].N, S["par"].delta_in)
    err = np.abs(slots - ref).max()
    say(f"[bootstrap] max |error| against the input's decryption: {err:.3g}")
    assert err < 1e-3
    out2 = boot.run(B.View(x))
    st.sync()
    got2 = out2.h.buf.download((2, ctx.rows, ctx.n), offset=out2.h.off, words=ctx.ct_words)
    assert (got2[:, : out.top + 1] == got[:, : out.top + 1]).all(), "the rerun gives the same words"


@pytest.mark.parametrize("lanes", [1, 2, "pair"])
def test_bootstrap_graph_replay(lanes):
    """The whole bootstrap captured into one HIP graph (the composite's operations never allocate, synchronise or read
    device data on the host once a first run has filled the buffer pool and the constants) and replayed three times,
    with the output cleared and eager work on the same buffers between the replays: every replay equals the eager run
    word for word."""
    say(f"[bootstrap graph] N=2^12, {lanes} EvalMod lane(s): capture, 3 replays vs the eager run")
    S = setup_oracle(fused=False)
    rng = np.random.default_rng(11)
    z, ct, me = input_ct(S, rng)
    ctx, keys, relin, st, ops, boot = gpu_boot(S, lanes)
    x = pa.DevBuf.from_array(ct)
    out = boot.run(B.View(x))
    st.sync()
    want = out.h.buf.download((2, ctx.rows, ctx.n), offset=out.h.off, words=ctx.ct_words)
    graph = pa.Graph(st, lambda: boot.run(B.View(x)))
    zeros = np.zeros(ctx.ct_words, np.uint32)
    for rep in range(3):
        out.h.buf.upload(zeros, offset=out.h.off)
        other = ctx.ct_buf()
        ctx.rotate(keys, 0, x, boot.T, other, st)  # eager work through the same context's workspace
        st.sync()
        graph.launch(st)
        st.sync()
        got = out.h.buf.download((2, ctx.rows, ctx.n), offset=out.h.off, words=ctx.ct_words)
        say(f"[bootstrap graph] replay {rep}")
        assert (got[:, : out.top + 1] == want[:, : out.top + 1]).all(), f"replay {rep} == eager"
