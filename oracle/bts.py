"""CPU restatement of the bootstrap's raise kernels (ModRaise, the small-integer scalings): part of the ORACLE of this
repository's tests.

Test infrastructure only. Nothing in the product library (perseus_amd/) imports this module; only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg use it, to check the GPU's results against.

Semantics: crates/pc-kernels/kernels/args.cuh ModRaiseArgs / SmallIntArgs / SmallInt1Args :665-709, :890-907, and the
host twins crates/pc-gpu/src/bts/raise.rs:159-215 (small_int_host), :279-292 (small_int1_host). The multi-word
integers are Python integers in numpy object arrays, so nothing here is bounded by a word size.
"""
import numpy as np


def mod_raise(q, rows, d, r0, r1, qhatinv, qhat):
    """One polynomial's coefficient rows [>= r1][N] (row t mod q[t]): rows t in [r0, r1) become
    sum_{k < d} lift_t([x_k qhatinv[k]]_{q_k}) qhat[k][t] mod q_t, lift_t(y) = (y - q_k if y > q_k / 2 else y) mod q_t
    (bts.cuh:14-33). Returns the new rows [r1 - r0][N]."""
    out = []
    for t in range(r0, r1):
        qt = int(q[t])
        acc = np.zeros(rows.shape[-1], object)
        for k in range(d):
            qk = int(q[k])
            y = rows[k].astype(object) * int(qhatinv[k]) % qk
            lift = np.where(y > qk // 2, y - qk, y) % qt
            acc = (acc + lift * (int(qhat[k][t]) % qt)) % qt
        out.append(acc.astype(np.uint32))
    return np.stack(out)


def small_int(q_src, rows, out_primes, r_words=None):
    """One polynomial (bts.cuh:56-170; raise.rs:159-215): X from the source rows [k][N] by Garner's mixed radix, centred
    against Q_k / 2 (X > floor(Q_k / 2) -> negative, magnitude Q_k - X); with the reciprocal R = sum_w r_words[w] 2^(32 w)
    the magnitude becomes floor((|X| R + 2^191) / 2^192); each output row = sign(X) |.| mod p. Returns [nout][N]."""
    k = len(q_src)
    q_src = [int(x) for x in q_src]
    v = []
    for i in range(k):
        dgt = rows[i].astype(object) % q_src[i]
        for j in range(i):
            dgt = (dgt - v[j]) * pow(q_src[j], -1, q_src[i]) % q_src[i]
        v.append(dgt)
    x = v[k - 1]
    for i in range(k - 2, -1, -1):
        x = x * q_src[i] + v[i]
    big = 1
    for p in q_src:
        big *= p
    neg = x > big // 2
    mag = np.where(neg, big - x, x)
    if r_words is not None:
        r = sum(int(w) << (32 * i) for i, w in enumerate(r_words))
        mag = (mag * r + (1 << 191)) >> 192
    out = []
    for p in out_primes:
        m = mag % int(p)
        out.append(np.where(neg & (m != 0), int(p) - m, m).astype(np.uint64))
    return np.stack(out)


def small_int1(q0, mc, sh, row0, out_primes):
    """One polynomial (bts.cuh:173-190; raise.rs:279-292): x = row 0 centred against q0, q = floor((|x| mc + 2^(sh-1)) /
    2^sh), each output row = sign(x) q mod p. Returns [nout][N]."""
    v = row0.astype(object)
    neg = v > int(q0) // 2
    mag = np.where(neg, int(q0) - v, v)
    qv = (mag * int(mc) + (1 << (sh - 1))) >> sh
    out = []
    for p in out_primes:
        m = qv % int(p)
        out.append(np.where(neg & (m != 0), int(p) - m, m).astype(np.uint64))
    return np.stack(out)
