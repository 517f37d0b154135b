"""Host-side tables of the bootstrap's raise kernels (crates/pc-gpu/src/bts/raise.rs): the composite ModRaise's CRT
constants, the small-integer scaling table with its 2^192 fixed-point reciprocal (computed the way x87 extended
precision rounds, raise.rs:30-93), and the one-prime scale mc / 2^sh (raise.rs:247-277). They fill the ABI structs of
perseus_amd.abi; the kernels run in libpchip.so."""
import struct

from . import abi

SI_MAXK, SI_MAXW, SI_MAXR, SI_SHIFT, SI_MAXOUT = 4, 8, 8, 192, 64


def div_rn64(num_exp, den):
    """2^num_exp / den rounded to nearest even at a 64-bit mantissa: (m, e) with m in [2^63, 2^64), value m 2^e
    (raise.rs:40-64)."""
    k = 127 - (64 - den.bit_length())
    q = (1 << k) // den
    while q >= 1 << 64:
        k -= 1
        q = (1 << k) // den
    r = (1 << k) - q * den
    m, e = q, num_exp - k
    if 2 * r > den or (2 * r == den and m & 1):
        m += 1
        if m == 1 << 64:
            m, e = 1 << 63, e + 1
    return m, e


def _f64_parts(c):
    bits = struct.unpack("<Q", struct.pack("<d", c))[0]
    exp, frac = (bits >> 52) & 0x7FF, bits & ((1 << 52) - 1)
    return (frac, -1074) if exp == 0 else (frac | (1 << 52), exp - 1075)


def reciprocal_words(c):
    """R = round(2^192 / D) for D = 1 / c, both quotients at x87 precision (raise.rs:66-93), as SI_MAXR 32-bit words."""
    if not (c > 0.0) or c != c or c == float("inf"):
        raise ValueError(f"scaling constant {c} must be positive")
    mc, ec = _f64_parts(c)
    dm, de = div_rn64(-ec, mc)
    vm, sh = div_rn64(SI_SHIFT - de, dm)
    if sh < 0 or sh + 64 > 32 * SI_MAXR:
        raise ValueError(f"reciprocal shift {sh} outside the table (constant {c})")
    r = vm << (sh % 32)
    w0 = sh // 32
    out = [0] * SI_MAXR
    for i in range(4):
        if w0 + i < SI_MAXR:
            out[w0 + i] = (r >> (32 * i)) & 0xFFFFFFFF
    return out


def small_int_tab(src, out_rows, out_primes, c=None):
    """The SmallIntTab of sources `src` (primes below 2^31), outputs at prime ids `out_rows` of primes `out_primes`;
    c: scale by c (D = 1 / c), None: the centred lift only (raise.rs:97-156)."""
    if not src or len(src) > SI_MAXK or len(out_rows) > SI_MAXOUT or len(out_rows) != len(out_primes):
        raise ValueError(f"{len(src)} sources (<= {SI_MAXK}), {len(out_rows)} outputs (<= {SI_MAXOUT})")
    t = abi.SmallIntTab()
    t.k, t.nout = len(src), len(out_rows)
    for i, qi in enumerate(src):
        if qi >= 1 << 31:
            raise ValueError("source primes must be below 2^31")
        t.q[i] = qi
        for j in range(i):
            t.qinv[i][j] = pow(src[j] % qi, -1, qi)
    big = 1
    for qi in src:
        big *= qi
    words = []
    while big:
        words.append(big & 0xFFFFFFFF)
        big >>= 32
    t.nw = len(words) + 1
    if t.nw > SI_MAXW:
        raise ValueError("source product too wide")
    qk = 0
    for w, v in enumerate(words):
        t.Qk[w] = v
        qk |= v << (32 * w)
    half = qk >> 1
    for w in range(len(words)):
        t.Qkh[w] = (half >> (32 * w)) & 0xFFFFFFFF
    if c is not None:
        t.divide = 1
        r = reciprocal_words(c)
        for w, v in enumerate(r):
            t.R[w] = v
        nr = SI_MAXR
        while nr > 1 and r[nr - 1] == 0:
            nr -= 1
        t.nr = nr
    for o, (row, p) in enumerate(zip(out_rows, out_primes)):
        t.orow[o] = row
        for w in range(SI_MAXW + SI_MAXR):
            t.pow32[o][w] = pow(2, 32 * w, p)
    return t


def single_scale(c, q0):
    """c = mc 2^-sh exactly (the double's mantissa, trailing zeros stripped, sh >= 1), refused when round(c |x|) can
    leave 64 bits for |x| <= q0 / 2 (raise.rs:247-277)."""
    if not (c > 0.0) or c != c or c == float("inf"):
        raise ValueError(f"scaling constant {c} must be positive")
    mc, e = _f64_parts(c)
    while mc & 1 == 0 and e < -1:
        mc >>= 1
        e += 1
    while e > -1:
        if mc >> 63:
            raise ValueError(f"scaling constant {c} too large")
        mc <<= 1
        e -= 1
    sh = -e
    if sh > 127:
        raise ValueError(f"scaling constant {c} needs a shift of {sh} (> 127)")
    if ((q0 // 2) * mc + (1 << (sh - 1))) >> sh >= 1 << 64:
        raise ValueError(f"round(c |x|) leaves 64 bits for |x| <= q0/2 (c = {c})")
    return mc, sh


def mod_raise_consts(q, d):
    """The ModRaise tables of d source primes q[0..d-1] over every prime of q (raise.rs:461-480): qhatinv[k] =
    (Q_d / q_k)^-1 mod q_k, qhat[k][t] = Q_d / q_k mod q_t."""
    if not 1 <= d <= 4 or len(q) > 64:
        raise ValueError("1 <= d <= 4 sources, at most 64 rows")
    qhatinv, qhat = [0] * 4, [[0] * 64 for _ in range(4)]
    for k in range(d):
        hat = 1
        for j in range(d):
            if j != k:
                hat *= q[j]
        qhatinv[k] = pow(hat % q[k], -1, q[k])
        for t, qt in enumerate(q):
            qhat[k][t] = hat % qt
    return qhatinv, qhat
