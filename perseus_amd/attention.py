"""Encrypted attention scoring for a GPT-2-small-shaped decode step (12 heads of 64 dimensions, d_model 768, a KV cache
of 512 tokens): the keys K live encrypted in HBM, the query q is a plaintext, and the scores s[h][t] = sum_d q[h][d]
K[t][64 h + d] come out encrypted, one per slot. The operation sequence is the reference's scoring recipe
(crates/pc-gpu/src/ops.rs:927-951 mult_pt, crates/pc-gpu/src/rescale.rs:230-264, crates/pc-gpu/src/rotate.rs:924-992
rotate_and_sum): per ciphertext a plaintext product, a two-prime rescale back to the ciphertext's scale, and the
log-step rotate-and-sum over each 64-slot head block.

Packing (complex, two real vectors per ciphertext): N/2 = 2^15 slots hold 512 blocks of 64; ciphertext c carries heads
2c and 2c + 1, block (hl, t) = 256 hl + t for t < 256, its real part token t and its imaginary part token t + 256, slot
64 block + d the key's dimension d. The query plaintext repeats q[h] over its head's blocks (a real multiplier, so it
scales both parts alike). After the sums, slot 64 block holds s[h][t] + i s[h][t + 256]."""
import numpy as np

HEADS, HEAD_DIM, TOKENS = 12, 64, 512
BLOCK = HEAD_DIM
HEADS_PER_CT = 2
TOK_PER_PART = TOKENS // 2


def n_cts():
    return HEADS // HEADS_PER_CT


def key_slots(K, n):
    """The ciphertexts' slot vectors (N/2 complex each) of the key matrix K [TOKENS][HEADS * HEAD_DIM]."""
    assert n // 2 == HEADS_PER_CT * TOK_PER_PART * BLOCK, "the packing fills N/2 slots at N = 2^16"
    out = []
    for c in range(n_cts()):
        z = np.zeros(n // 2, np.complex128)
        for hl in range(HEADS_PER_CT):
            h = HEADS_PER_CT * c + hl
            blk = K[:, h * HEAD_DIM:(h + 1) * HEAD_DIM]  # [TOKENS][64]
            part = blk[:TOK_PER_PART] + 1j * blk[TOK_PER_PART:]
            z[hl * TOK_PER_PART * BLOCK:(hl + 1) * TOK_PER_PART * BLOCK] = part.reshape(-1)
        out.append(z)
    return out


def query_slots(q, n):
    """The plaintexts' slot vectors (real) of the query q [HEADS][HEAD_DIM], one per ciphertext."""
    out = []
    for c in range(n_cts()):
        z = np.zeros(n // 2, np.float64)
        for hl in range(HEADS_PER_CT):
            h = HEADS_PER_CT * c + hl
            z[hl * TOK_PER_PART * BLOCK:(hl + 1) * TOK_PER_PART * BLOCK] = np.tile(q[h], TOK_PER_PART)
        out.append(z)
    return out


def scores_from_slots(zs):
    """s [HEADS][TOKENS] from the decrypted, decoded slot vectors of the ciphertexts."""
    s = np.zeros((HEADS, TOKENS))
    for c, z in enumerate(zs):
        for hl in range(HEADS_PER_CT):
            h = HEADS_PER_CT * c + hl
            v = z[hl * TOK_PER_PART * BLOCK:(hl + 1) * TOK_PER_PART * BLOCK:BLOCK]
            s[h, :TOK_PER_PART] = v.real
            s[h, TOK_PER_PART:] = v.imag
    return s


# the ladder's radix 2^3: two rungs of seven rotations, each rung one ModUp shared by its seven key dots (measured on
# MI355X: 0.95 ms per scoring against 1.6 ms for the six-rung log ladder and 1.9 ms for one rung of 63)
RADIX_BITS = 3


def ladder_steps(radix_bits=RADIX_BITS):
    """The rotation steps the ladder over a 64-slot block takes: 1, 2, 4, ..., 32 rung by rung; with radix_bits r,
    rungs of 2^r - 1 summed rotations by j g (j < 2^r, g = 1, 2^r, 4^r, ...)."""
    if radix_bits <= 1:
        return [1 << k for k in range(6)]
    out, g = [], 1
    while g < BLOCK:
        n = min(radix_bits, (BLOCK // g).bit_length() - 1)
        out += [j * g for j in range(1, 1 << n)]
        g <<= n
    return out


def score(ctx, keys, ct, pt, top, out, tmp, stream, radix_bits=RADIX_BITS):
    """One ciphertext's scores: out = rotate_and_sum(rescale(ct pt)) over the head blocks at limb top - 2; keys holds
    the rotations of ladder_steps(radix_bits). ct is left untouched; out and tmp are single ciphertexts (tmp: the
    ladder's scratch)."""
    ctx.mul_plain(ct, pt, top, out, stream)
    ctx.rescale(out, top, 2, out, stream)
    ctx.rotate_and_sum(keys, out, top - 2, 1, BLOCK, out, tmp, stream, radix_bits=radix_bits)


def score_batch(ctx, keys, cts, pts, top, outs, tmp, stream, radix_bits=RADIX_BITS):
    """Every ciphertext's scores at once: cts, outs and tmp each K consecutive ciphertexts of one buffer (the ctx's
    k_max and k_rot at least K), pts the K plaintexts; the plaintext products (each ciphertext by its own plaintext),
    the two-prime rescale and the ladder as K-ciphertext launches (pcx_mul_plain_k, pcx_rescale_k,
    pcx_rotate_and_sum_k). The words of score() on each ciphertext."""
    K = len(pts)
    ctx.mul_plain_k(cts, pts, top, outs, stream)
    ctx.rescale(outs, top, 2, outs, stream, K=K)
    ctx.rotate_and_sum(keys, outs, top - 2, 1, BLOCK, outs, tmp, stream, radix_bits=radix_bits, K=K)


def score_streams(lanes, cts, pts, top, outs, main, radix_bits=RADIX_BITS):
    """The scorings of independent ciphertexts side by side: lane i = (context, keys, stream, tmp) takes ciphertexts
    i, i + len(lanes), ...; each lane has its own context (its own workspace), so the lanes' small kernels overlap on
    the chip. Ordered after the work already on `main`, and `main` waits for every lane."""
    from .engine import Event

    start = Event()
    start.record(main)
    ends = []
    for i, (ctx, keys, st, tmp) in enumerate(lanes):
        st.wait(start)
        for c in range(i, len(cts), len(lanes)):
            score(ctx, keys, cts[c], pts[c], top, outs[c], tmp, st, radix_bits)
        e = Event()
        e.record(st)
        ends.append(e)
    for e in ends:
        main.wait(e)
