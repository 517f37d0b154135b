"""CPU restatement of the EvalMod / plaintext-product element-wise kernels and of the composite rescale: part of the
ORACLE of this repository's tests.

Test infrastructure only. Nothing in the product library (perseus_amd/) imports this module; only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg use it, to check the GPU's results against.

Each function states one kernel of the reference's table over canonical residues with numpy uint64 arithmetic (every
product is reduced before it is summed, so any number of terms is exact). Arrays are ciphertext slices
[K][2 parts][n rows][N] whose row index is the prime id; `q` holds the primes of those rows. The semantics follow
crates/pc-kernels/kernels/args.cuh (the struct comments cited per function) and the host twin
crates/pc-host/src/elem.rs, crates/pc-host/src/rescale.rs.
"""
import numpy as np

U64 = np.uint64


def _q(q, n):
    return np.asarray(q[:n], U64).reshape(n, 1)


def _u(x):
    return np.asarray(x).astype(U64)


def _mul(a, b, q):
    return (_u(a) * _u(b)) % q


def _add(a, b, q):
    return (_u(a) + _u(b)) % q


def _sub(a, b, q):
    return (_u(a) + q - _u(b)) % q


def _row(v, n):
    """a per-row constant vector as a column"""
    return np.asarray(v[:n], U64).reshape(n, 1)


def _out(x):
    return x.astype(np.uint32)


def tensor(q, pairs, old=None, old_d2=None, acc=False, acc_d2=False, dbl=False, y=None, yc=None, ysub=False):
    """tensor / tensor_y / tensor_sum (args.cuh:356-389; em.cuh:12-78, :80-123; elem.rs:205-266): pairs = [(a, b)]
    of [K][2][n][N] ciphertexts -> (c0, c1, d2) = sum_j (a0 b0, a0 b1 + a1 b0, a1 b1); acc: (c0, c1) += old's parts,
    acc_d2: d2 += old_d2; dbl: all three doubled after the adds; y, yc: (c0, c1) +-= y yc[row] (tensor_y, after the
    doubling). Returns c0, c1, d2 each [K][n][N]."""
    a0 = pairs[0][0]
    n = a0.shape[2]
    qq = _q(q, n)
    s0 = np.zeros(a0[:, 0].shape, U64)
    s1, s2 = s0.copy(), s0.copy()
    for a, b in pairs:
        s0 = _add(s0, _mul(a[:, 0], b[:, 0], qq), qq)
        s1 = _add(s1, _add(_mul(a[:, 0], b[:, 1], qq), _mul(a[:, 1], b[:, 0], qq), qq), qq)
        s2 = _add(s2, _mul(a[:, 1], b[:, 1], qq), qq)
    if acc:
        s0, s1 = _add(s0, old[:, 0], qq), _add(s1, old[:, 1], qq)
    if acc_d2:
        s2 = _add(s2, old_d2, qq)
    if dbl:
        s0, s1, s2 = _add(s0, s0, qq), _add(s1, s1, qq), _add(s2, s2, qq)
    if y is not None:
        c = _row(yc, n)
        m0, m1 = _mul(y[:, 0], c, qq), _mul(y[:, 1], c, qq)
        s0 = _sub(s0, m0, qq) if ysub else _add(s0, m0, qq)
        s1 = _sub(s1, m1, qq) if ysub else _add(s1, m1, qq)
    return _out(s0), _out(s1), _out(s2)


def md_epilogue(q, dst, x, t, binv, k=None, dbl=False):
    """md_epilogue (args.cuh:438-447; em.cuh:383-400; elem.rs:406-427): for both parts dst = f (dst + (x - t) binv)
    [+ k[row] on part 0, reduced once], f = 2 when dbl."""
    n = dst.shape[2]
    qq = _q(q, n)
    r = _add(dst, _mul(_sub(x, t, qq), _row(binv, n), qq), qq)
    if dbl:
        r = _add(r, r, qq)
    if k is not None:
        r[:, 0] = _add(r[:, 0], _row(k, n) % qq, qq)
    return _out(r)


def md_epilogue_to(q, a, x, t, binv, sub=False):
    """md_epilogue_to (args.cuh:449-456; em.cuh:403-418): dst = a +- (x - t) binv on both parts."""
    n = a.shape[2]
    qq = _q(q, n)
    v = _mul(_sub(x, t, qq), _row(binv, n), qq)
    return _out(_sub(a, v, qq) if sub else _add(a, v, qq))


def wsum(q, srcs, w, k=None):
    """wsum / wsum_k / one output of wsum_multi (args.cuh:458-489; em.cuh:420-480; elem.rs:450-517):
    out = sum_j w[j][row] src_j on both parts [+ k[row] on part 0, reduced once]; w: [nsrc][n]."""
    n = srcs[0].shape[2]
    qq = _q(q, n)
    r = np.zeros(srcs[0].shape, U64)
    for j, s in enumerate(srcs):
        r = _add(r, _mul(s, _row(w[j], n), qq), qq)
    if k is not None:
        r[:, 0] = _add(r[:, 0], _row(k, n) % qq, qq)
    return _out(r)


def add_const(q, x, k):
    """add_const (args.cuh:491-498; em.cuh:496-506): part 0 += k[row], reduced once."""
    n = x.shape[2]
    qq = _q(q, n)
    r = _u(x).copy()
    r[:, 0] = _add(r[:, 0], _row(k, n) % qq, qq)
    return _out(r)


def mul_add_n(q, terms, y=None, mode=0):
    """mul_table / mul_add / mul_add_n (args.cuh:500-528; em.cuh:508-565; elem.rs:532-636): s = sum_j x_j t_j with
    t_j a table [n][N] shared by the K ciphertexts and both parts; out = s (no y), y + s (mode 0), y - s (1), s - y (2)."""
    n = terms[0][0].shape[2]
    qq = _q(q, n)
    s = np.zeros(terms[0][0].shape, U64)
    for x, t in terms:
        s = _add(s, _mul(x, np.asarray(t[:n], U64)[None, None], qq), qq)
    if y is None:
        return _out(s)
    return _out(_add(y, s, qq) if mode == 0 else _sub(y, s, qq) if mode == 1 else _sub(s, y, qq))


def combine(q, x, tmp, alpha):
    """rescale_combine / rescale_combine_to (args.cuh:565-579; rescale.cuh:63-77; em.cuh:482-494):
    alpha_i x_i + tmp_i on both parts."""
    n = x.shape[2]
    qq = _q(q, n)
    return _out(_add(_mul(x, _row(alpha, n), qq), tmp, qq))


def ew_many(q, a, b=None, c=None):
    """one polynomial of ew_many (args.cuh:162-170; elem.rs:109-129): a (+ b) (+ c), rows [n][N]."""
    n = a.shape[0]
    qq = _q(q, n)
    r = _u(a)
    for z in (b, c):
        if z is not None:
            r = _add(r, z, qq)
    return _out(r)


def submul_many(q, a, b, t):
    """one polynomial of submul_many (args.cuh:172-182; elem.rs:131-143): (a - b) t, rows [n][N]."""
    n = a.shape[0]
    qq = _q(q, n)
    return _out(_mul(_sub(a, b, qq), np.asarray(t[:n], U64), qq))


# ----------------------------------------------------------------------------------------------- composite rescale
def inv(a, m):
    a %= m
    return pow(a, -1, m) if a else 0


def rescale_consts(q, top, ndrop):
    """The host constants of a drop of ndrop primes from limb `top` (crates/pc-gpu/src/rescale.rs:118-160 from
    crates/pc-core/src/scale.rs:196-208): qlql[l][i] = -q_l^-1 mod q_i, q_inv[a][i] = q_a^-1 mod q_i.
    ndrop 1 (a = top):            A_i = qlql[a][i], alpha_i = q_inv[a][i]
    ndrop 2 (a = top, b = top-1): A_i = q_inv[b][i] qlql[a][i], B_i = qlql[b][i], alpha_i = q_inv[b][i] q_inv[a][i],
                                  qinv_ab = q_inv[a][b], C_ab = qlql[a][b]
    and qam / qbm = q_a / q_b mod q_i, over rows i < top + 1 - ndrop."""
    q = [int(v) for v in q]
    a, b = top, top - 1

    def qlql(l, i):
        v = inv(q[l], q[i])
        return q[i] - v if v else 0

    rows = top + 1 - ndrop
    c = {"qam": [q[a] % q[i] for i in range(rows)]}
    if ndrop == 1:
        c["A"] = [qlql(a, i) for i in range(rows)]
        c["alpha"] = [inv(q[a], q[i]) for i in range(rows)]
        c["B"], c["qbm"], c["qinv_ab"], c["C_ab"] = [0] * rows, [0] * rows, 0, 0
    else:
        c["A"] = [inv(q[b], q[i]) * qlql(a, i) % q[i] for i in range(rows)]
        c["B"] = [qlql(b, i) for i in range(rows)]
        c["alpha"] = [inv(q[b], q[i]) * inv(q[a], q[i]) % q[i] for i in range(rows)]
        c["qbm"] = [q[b] % q[i] for i in range(rows)]
        c["qinv_ab"], c["C_ab"] = inv(q[a], q[b]), qlql(a, b)
    return c


def _lift(y, qo, qi):
    """the centred representative of y (mod qo) reduced mod qi (rescale.cuh:12-24)"""
    y = _u(y)
    yr = y % qi
    return np.where(y > U64(qo >> 1), (yr + qi - U64(qo % qi)) % qi, yr)


def rescale_coef(q, ya, yb, top, ndrop, consts, ca=1, cb=1):
    """rescale_coef (args.cuh:531-552; rescale.cuh:26-61): the correction rows tmp_i, i < top + 1 - ndrop, of one
    polynomial from its tops in coefficient form (ya = row top, yb = row top - 1); ca / cb scale the tops first
    (when ca != 1). Returns (tmp [rows][N], y') with y' the ndrop-2 second source (None for ndrop 1)."""
    q = [int(v) for v in q]
    a, b = top, top - 1
    ya = _u(ya)
    if ca != 1:
        ya = (ya * U64(ca % q[a])) % U64(q[a])
    yp = None
    if ndrop == 2:
        yb = _u(yb)
        if ca != 1:
            yb = (yb * U64(cb % q[b])) % U64(q[b])
        qb = U64(q[b])
        yp = ((yb * U64(consts["qinv_ab"])) % qb + (_lift(ya, q[a], qb) * U64(consts["C_ab"])) % qb) % qb
    rows = top + 1 - ndrop
    tmp = np.zeros((rows, ya.shape[-1]), U64)
    for i in range(rows):
        qi = U64(q[i])
        w = (_lift(ya, q[a], qi) * U64(consts["A"][i])) % qi
        if ndrop == 2:
            w = (w + (_lift(yp, q[b], qi) * U64(consts["B"][i])) % qi) % qi
        tmp[i] = w
    return tmp.astype(np.uint32), None if yp is None else yp.astype(np.uint32)


def rescale(oc, q, x, top, ndrop, fold=None):
    """The composite one-pass rescale of ciphertexts x [K][2][rows][N] (eval form) from limb `top` by ndrop primes
    (crates/pc-gpu/src/rescale.rs:318-400 `composite_from`, :402-440 `single`): INTT the tops, rescale_coef, NTT the
    corrections, x_i = alpha_i x_i + tmp_i (alpha_i c_i with a fold c [by prime id]: the rescale of c x). oc: the
    twin context (its ntt_fwd / ntt_inv over rows and prime ids); top >= 1. Returns the new rows [K][2][top + 1 - ndrop][N]."""
    K = x.shape[0]
    c = rescale_consts(q, top, ndrop)
    rows = top + 1 - ndrop
    alpha = list(c["alpha"])
    ca = cb = 1
    if fold is not None:
        ca, cb = int(fold[top]) % int(q[top]), int(fold[top - 1]) % int(q[top - 1])
        alpha = [alpha[i] * (int(fold[i]) % int(q[i])) % int(q[i]) for i in range(rows)]
    out = np.zeros((K, 2, rows, x.shape[-1]), np.uint32)
    for k in range(K):
        for part in range(2):
            tops = oc.ntt_inv(x[k, part, top - 1:top + 1].copy(), [top - 1, top])
            tmp, _ = rescale_coef(q, tops[1], tops[0], top, ndrop, c, ca, cb)
            tmp = oc.ntt_fwd(tmp, list(range(rows)))
            out[k, part] = combine(q, x[k:k + 1, part:part + 1, :rows], tmp[None, None], alpha)[0, 0]
    return out


# ----------------------------------------------------------------------------------------------- encryption
def encrypt(q, a, s, e, m=None):
    """encrypt (args.cuh:613-628; encrypt.cuh:10-31): limb l (prime id l) of c0 = e + m - a s, with a the "ENCA"
    expander rows (twin.expand_row with w13 = the nonce), all [nl][N] in the evaluation domain."""
    n = a.shape[0]
    qq = _q(q, n)
    em_ = _u(e) if m is None else _add(e, m, qq)
    return _out(_sub(em_, _mul(a, s, qq), qq))


# ----------------------------------------------------------------------------------------------- BSGS plaintext dot
def ptidx(o, enc):
    """a diagonal's compact index of slot o (arith.cuh:242-244): o >> (enc & 0xFF) when enc >> 24 == 0x7F, else o & enc"""
    o = np.asarray(o, np.uint64)
    if enc >> 24 == 0x7F:
        return o >> np.uint64(enc & 0xFF)
    return o & np.uint64(enc)


def pt_dot(q, rot, pts, bstep, gstep, npts, enc, prows):
    """pt_dot (args.cuh:184-198; elem.cuh:83-118; elem.rs:145-193): rot [K][bstep][2][n][N] over rows with primes q[r],
    pts[d] [rows][ptw] read at row prows[r] and index ptidx(i, enc) -> res [K][gstep][2][n][N] with
    res[c][j] = sum_{b < bstep, bstep j + b < npts} rot[c][b] pt_{bstep j + b}."""
    K, _, _, n, N = rot.shape
    qq = _q(q, n)
    idx = ptidx(np.arange(N), enc).astype(np.int64)
    out = np.zeros((K, gstep, 2, n, N), np.uint32)
    for j in range(gstep):
        acc = np.zeros((K, 2, n, N), U64)
        for b in range(bstep):
            d = bstep * j + b
            if d >= npts:
                break
            w = np.stack([np.asarray(pts[d][prows[r]], U64)[idx] for r in range(n)])
            acc = _add(acc, _mul(rot[:, b], w[None, None], qq), qq)
        out[:, j] = _out(acc)
    return out


# ----------------------------------------------------------------------------------------------- subring switch
def pack_split(x, sub):
    """pack_split (args.cuh:230-241; ks.cuh:909-921; crates/pc-host/src/ks.rs:364-381): rows [nrows][N] of one
    polynomial -> digits [sub][nrows][N], digit j keeping the coefficients at exponents = j mod sub."""
    N = x.shape[-1]
    cls = np.arange(N) % sub
    return np.stack([np.where(cls == j, x, 0).astype(np.uint32) for j in range(sub)])


def pack_dot(q, dig, kb, ka, c0=None, pmod=None, nq=0):
    """pack_dot (args.cuh:243-259; ks.cuh:923-947; crates/pc-host/src/ks.rs:383-405): digits, key b and key a
    [sub][n][N] over rows of primes q -> (s0, s1) [n][N]: s1 = sum_j D_j a_j, s0 = sum_j D_j b_j, plus pmod[y] c0 on
    the first nq rows."""
    n = dig.shape[1]
    qq = _q(q, n)
    s0 = np.zeros(dig.shape[1:], U64)
    s1 = s0.copy()
    for j in range(dig.shape[0]):
        s0 = _add(s0, _mul(dig[j], kb[j], qq), qq)
        s1 = _add(s1, _mul(dig[j], ka[j], qq), qq)
    if nq:
        s0[:nq] = _add(s0[:nq], _mul(c0[:nq], _row(pmod, nq), qq[:nq]), qq[:nq])
    return _out(s0), _out(s1)


# ----------------------------------------------------------------------------------------------- coeff_sum
def coeff_residues(rows, scale, q):
    """round(rows * scale) (float32 rows widened to float64, half to even) as residues [len(q)][n][N]; a product of
    magnitude 9.2e18 or more becomes +-2^62 and is counted once per limb (args.cuh:906-911;
    crates/pc-host/src/coeffrows.rs:11-27). Returns (residues, overflow count)."""
    x = np.asarray(rows, np.float32).astype(np.float64) * float(scale)
    big = ~(np.abs(x) < 9.2e18)
    m = np.where(big, np.where(x < 0, -(2.0 ** 62), 2.0 ** 62), np.rint(np.where(big, 0.0, x))).astype(np.int64)
    mag = np.abs(m).astype(U64)
    out = []
    for p in q:
        v = mag % U64(p)
        v = np.where((m < 0) & (v != 0), U64(p) - v, v)
        out.append(v.astype(np.uint32))
    return np.stack(out), int(big.sum()) * len(q)


def coeff_sum(q, rows, scale, cts, ntt, out=None):
    """coeff_sum (args.cuh:906-927; coeffrows.rs:30-80): out (+)= sum_r ct_r NTT(round(rows_r scale)) over limbs
    l < len(q) (prime id l). cts [n][2][L][N]; ntt(rows [L][N], ids) the forward transform. Returns (out, overflow)."""
    res, ovf = coeff_residues(rows, scale, q)
    L, n, N = res.shape
    qq = np.asarray(q, U64)[:, None]
    acc = np.zeros((2, L, N), U64) if out is None else np.asarray(out, U64).copy() % qq
    for r in range(n):
        pt = np.asarray(ntt(np.ascontiguousarray(res[:, r]), list(range(L))), U64)
        for part in range(2):
            acc[part] = (acc[part] + pt * np.asarray(cts[r][part], U64) % qq) % qq
    return acc.astype(np.uint32), ovf


# ----------------------------------------------------------------------------------------------- tensor_seeded
PACK_BITS = 28


def pack28(rows):
    """rows [n][N] of values below 2^28 as little-endian 28-bit streams, (N 28 + 31) / 32 words per row
    (args.cuh:412-413)"""
    rows = np.asarray(rows, U64)
    n, N = rows.shape
    words = (N * PACK_BITS + 31) // 32
    out = np.zeros((n, words + 1), U64)
    for i in range(N):
        bit = PACK_BITS * i
        w, sh = bit >> 5, bit & 31
        v = rows[:, i] << U64(sh)
        out[:, w] |= v & U64(0xFFFFFFFF)
        out[:, w + 1] |= v >> U64(32)
    return out[:, :words].astype(np.uint32)


def tensor_seeded(q, c0s, seeds, bsets, acc=0, old=None, old_d2=None, cts_row=None):
    """tensor_seeded (args.cuh:407-436; crates/pc-host/src/elem.rs:345-404): first operands o < nout, j < npairs given
    by their c0 rows c0s[o][j] [n][N] (the words as stored) and row seeds seeds[o][j] [n][8], their c1 rows drawn by
    cts_row(seed, p, N); second-operand sets bsets[q][j] [2][n][N]. Output m = q nout + o: (c0, c1, d2) =
    sum_j (x0 y0, x0 y1 + x1 y0, x1 y1) mod p; acc nonzero adds the old c0, c1, bit 1 the old d2.
    Returns (out [M][2][n][N], d2 [M][n][N])."""
    nout, npairs = len(c0s), len(c0s[0])
    n, N = np.asarray(c0s[0][0]).shape
    qq = np.asarray(q[:n], U64)[:, None]
    outs, d2s = [], []
    for bs in bsets:
        for o in range(nout):
            s0 = np.zeros((n, N), U64)
            s1 = np.zeros((n, N), U64)
            s2 = np.zeros((n, N), U64)
            for j in range(npairs):
                x0 = np.asarray(c0s[o][j], U64) % qq
                x1 = np.stack([np.asarray(cts_row(seeds[o][j][r], int(q[r]), N), U64) for r in range(n)])
                y0, y1 = np.asarray(bs[j][0], U64), np.asarray(bs[j][1], U64)
                s0 = (s0 + x0 * y0 % qq) % qq
                s1 = (s1 + x0 * y1 % qq + x1 * y0 % qq) % qq
                s2 = (s2 + x1 * y1 % qq) % qq
            m = len(outs)
            if acc:
                s0 = (s0 + np.asarray(old[m][0], U64)) % qq
                s1 = (s1 + np.asarray(old[m][1], U64)) % qq
            if acc & 2:
                s2 = (s2 + np.asarray(old_d2[m], U64)) % qq
            outs.append(np.stack([s0, s1]).astype(np.uint32))
            d2s.append(s2.astype(np.uint32))
    return np.stack(outs), np.stack(d2s)
