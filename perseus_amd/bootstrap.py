"""Full-slot CKKS bootstrap (N/2 complex slots): ModRaise -> CoeffToSlot -> EvalMod -> SlotToCoeff, the composite of
the reference's dense route (crates/pc-gpu/src/bts/dense.rs:1-9: mod_raise, CtS x4 as BSGS linear transforms, EvalMod
as a Chebyshev series plus double angles on the real and imaginary parts, StC x3), built on this engine's device
operations. The constants are this module's own (host, float64); the linear-transform factors follow the published
special FFT of CKKS (the decoding map z_j = sum_i w_i zeta^(5^j i) factored into log2(N/2) butterfly layers, the
factorisation OpenFHE's collapsed FFT also uses: crates/pc-core/src/bts_setup.rs:366-435 CoeffEncodingOneLevel /
CoeffDecodingOneLevel).

Scale bookkeeping. Every ciphertext carries its scale as a float (the slot values are decode(P) / scale). A linear
transform level encodes its diagonals at scale q_a q_b g (q_a q_b the two primes the rescale after it drops, g the
level's gain), so the rescale leaves the values as transformed and multiplies the scale by g exactly. In EvalMod every
addition joins ciphertexts of the same scale: a term that would arrive at another scale is first multiplied by an
integer constant chosen for the target scale and rescaled (the targets are propagated top-down through the Chebyshev
evaluation, as Lattigo's polynomial evaluator does), so no scale mismatch ever enters a sum.

The composite is written against an operations object (`ops`): `GpuOps` below runs it on the device through the
engine; the tests run the same composite on the oracle's operations and compare the words.
"""
import math

import numpy as np

from . import bts_setup as S

# ----------------------------------------------------------------------------------------------- linear transforms


class LtPlan:
    """One linear-transform stage as the route evaluates it: a collapsed-FFT stage of the reference's factors in
    FIDESlib's layout (bts_setup.FidesStage): y = sum_j rot(sum_i pts[j][i] rot(x, baby[i]), giant[j]) with
    baby = rot_in (baby[0] = 0: the unrotated input), giant = rot_out, pts[j][i] the plaintext slot vector of diagonal
    B j + i (None past the stage's diagonals or where it is zero)."""

    def __init__(self, st, n):
        self.n = n
        self.B, self.G = st.b_step, st.g_step
        self.baby = [int(x) for x in st.rot_in]
        self.giant = [int(x) for x in st.rot_out]
        assert self.baby[0] == 0, "the first baby step is the unrotated input"
        self.pts = []
        for j in range(self.G):
            row = []
            for i in range(self.B):
                d = self.B * j + i
                v = st.pts[d] if d < st.num_diags else None
                row.append(None if v is None or not np.any(v) else np.asarray(v, np.complex128))
            self.pts.append(row)

    def apply(self, x):
        """plain evaluation in the stage's BSGS order (the check of the layout)"""
        rots = [np.roll(x, -b) for b in self.baby]
        y = np.zeros(self.n, complex)
        for j in range(self.G):
            acc = np.zeros(self.n, complex)
            for i in range(self.B):
                if self.pts[j][i] is not None:
                    acc += self.pts[j][i] * rots[i]
            y += np.roll(acc, -self.giant[j])
        return y

    def steps(self):
        """the rotation steps the stage takes (babies, then giants), reduced to (0, n)"""
        out = []
        for r in self.baby[1:] + self.giant:
            r %= self.n
            if r and r not in out:
                out.append(r)
        return out


def lt_plans(N, budget):
    """The CoeffToSlot and SlotToCoeff stages of the full-slot bootstrap at ring degree N: the reference's factors
    (bts_setup.cts_stc_factors with scale_enc = scale_dec = 1, its dense route's call, crates/pc-gpu/src/bts/
    dense.rs:83) in FIDESlib's layout, CtS in evaluation order. Returns (cts plans, stc plans, the CtS stages' total
    gain). The CtS stages compose to n brev(U0^-1) (OpenFHE's unnormalised inverse: each stage carries 2^layers), the
    StC stages to U0 brev, the decoding map, exactly."""
    n = N // 2
    f = S.cts_stc_factors(N, n, list(budget), [0, 0], 1.0, 1.0)
    cts, stc, _acc = f.fides_layout()
    return [LtPlan(st, n) for st in cts], [LtPlan(st, n) for st in stc], float(n)


# ----------------------------------------------------------------------------------------------- Chebyshev series


def cheb_split(c, g):
    """p = q T_g + r for p = sum_k c_k T_k of degree < 2g: T_{g + j} = 2 T_g T_j - T_{g - j}."""
    c = list(c)
    r = c[:g] + [0.0] * max(0, g - len(c))
    q = [0.0] * max(1, len(c) - g)
    for j in range(len(c) - g):
        v = c[g + j]
        if j == 0:
            q[0] += v
        else:
            q[j] += 2 * v
            r[g - j] -= v
    return np.array(q), np.array(r)


def cheb_eval(c, u):
    return np.polynomial.chebyshev.chebval(u, c)


class EvalModPlan:
    """The reference's EvalMod series (bts_setup.evalmod_k32_low: K = 32, degree 59, 3 double angles, the prefactor
    (2 pi)^(-1/8)) with its double-angle constants (bts_setup.double_angle_scalar): on u = y / K, the series
    a cos(2 pi (K u - 1/4) / 8), then x -> 2 x^2 - (2 pi)^(-2^(j - 3)) three times, reads sin(2 pi K u) / (2 pi).
    c holds the series with c0 halved: the reference's tables keep the evaluator convention (c0 / 2 + sum c_k T_k),
    this module's Chebyshev evaluation the plain sum; halving is exact."""

    def __init__(self):
        self.K, self.r = S.EVALMOD_K32, S.EVALMOD_K32_LOW_DA_ITS
        self.table = S.evalmod_k32_low()
        self.c = np.array([self.table[0] / 2.0] + list(self.table[1:]))
        self.deg = len(self.c) - 1
        self.scalars = [S.double_angle_scalar(j, self.r) for j in range(1, self.r + 1)]

    def plain(self, u):
        h = cheb_eval(self.c, u)
        for sc in self.scalars:
            h = 2 * h * h + sc
        return h


# ----------------------------------------------------------------------------------------------- parameters


class Params:
    """Bootstrap shape: slots n = N/2; the CtS / StC level budgets (OpenFHE's levelBudget: the collapsed FFT's stage
    counts, [4, 3] in the reference's dense route); the input's message scale and the EvalMod input's target scale.
    EvalMod is the reference's K = 32 series (EvalModPlan); the output scale is whatever the chain leaves."""

    def __init__(self, logn, budget=(4, 3), delta_in=2.0 ** 25, target=2.0 ** 60):
        self.logn, self.N, self.n = logn, 1 << logn, 1 << (logn - 1)
        self.budget = (min(budget[0], logn - 1), min(budget[1], logn - 1))
        self.K, self.r = S.EVALMOD_K32, S.EVALMOD_K32_LOW_DA_ITS
        self.delta_in, self.target = delta_in, target

    def levels_used(self):
        """composite (two-prime) levels the bootstrap consumes after ModRaise"""
        return self.budget[0] + 7 + self.r + self.budget[1]


def simulate(P, par, em=None):
    """Plain float simulation of the bootstrap's algorithm on an integer coefficient vector P (= m + q0 I after the raise,
    here given directly as P / q0): the reference's stages in FIDESlib's layout, the EvalMod series on the real and
    imaginary parts, the StC stages; returns the output slot values, the decoding of sin(2 pi P / q0) / (2 pi), i.e. of
    m / q0 when |m| << q0 -- the check that the factors, the layout and the EvalMod series compose to the bootstrap."""
    from .encoding import decode

    em = em or EvalModPlan()
    cts, stc, gain = lt_plans(par.N, par.budget)
    x = decode(P, par.N, 1.0) / (2.0 * par.K * gain)
    for p in cts:
        x = p.apply(x)
    re, im = x + np.conj(x), -1j * (x - np.conj(x))
    w = em.plain(re.real) + 1j * em.plain(im.real)
    for p in stc:
        w = p.apply(w)
    return w


# ----------------------------------------------------------------------------------------------- host encoding


def residues(f, primes):
    """Exact residues [len(primes)][N] (u32) of the integers nearest the float coefficients f (|f| < 2^85): f rounded,
    split f = a 2^32 + b with both parts exact in float64, then (a mod p) (2^32 mod p) + b mod p in int64."""
    f = np.rint(np.asarray(f, np.float64))
    a = np.floor(f / 4294967296.0)
    b = (f - a * 4294967296.0).astype(np.int64)
    a = a.astype(np.int64) if np.abs(a).max(initial=0) < 2.0 ** 62 else None
    assert a is not None, "coefficient beyond 2^85"
    out = np.empty((len(primes), f.shape[-1]), np.uint32)
    for r, p in enumerate(primes):
        p = int(p)
        out[r] = ((a % p) * ((1 << 32) % p) % p + b % p) % p
    return out


def encode_rows(z, N, scale, primes):
    """The plaintext of slot vector z (N/2 complex values) at `scale`, as coefficient residue rows over `primes`."""
    from .encoding import encode

    return residues(encode(z, N, scale), primes)


def compact_shift(rows, cap=12):
    """The largest s <= cap with every nonzero coefficient of the residue rows at an index divisible by 2^s
    (crates/pc-gpu/src/bts/cts.rs:277-289). Such a polynomial is one in X^(2^s): its evaluation rows, in the
    transforms' bit-reversed order, are constant on aligned blocks of 2^s words, so a diagonal is kept at width
    N / 2^s and read at index i >> s."""
    nz = np.flatnonzero(np.any(np.asarray(rows) != 0, axis=0))
    if nz.size == 0:
        return cap
    g = int(np.bitwise_or.reduce(nz))
    return cap if g == 0 else min(cap, (g & -g).bit_length() - 1)


def compact_rows(rows, s):
    """evaluation rows [n][N] constant on aligned blocks of 2^s words -> their [n][N >> s] block values; raises if a
    block is not constant"""
    rows = np.asarray(rows)
    if s == 0:
        return rows
    n, N = rows.shape
    blk = rows.reshape(n, N >> s, 1 << s)
    if not (blk == blk[:, :, :1]).all():
        raise ValueError(f"evaluation rows not constant on blocks of 2^{s} words")
    return np.ascontiguousarray(blk[:, :, 0])


def int_rows(k, primes):
    """An integer constant (any size, any sign) as residues per prime (Python ints)."""
    return [int(k) % int(p) for p in primes]


# ----------------------------------------------------------------------------------------------- scale-tracked evaluator


class Ct:
    """A ciphertext handle of the operations object, its top limb and its scale (slot values = decode / scale)."""
    __slots__ = ("h", "top", "scale")

    def __init__(self, h, top, scale):
        self.h, self.top, self.scale = h, top, scale


class Evaluator:
    def __init__(self, ops, primes):
        self.ops, self.q = ops, [int(p) for p in primes]

    def qq(self, top):
        """the two primes the rescale from `top` drops"""
        return float(self.q[top]) * float(self.q[top - 1])

    def mul(self, a, b, twice=False):
        """a b, or 2 a b (twice: the doubling folded into the product, the words of mul(double(a), b))"""
        t = min(a.top, b.top)
        out = self.ops.alloc()
        self.ops.mul_relin_rescale(out, a.h, b.h, t, twice)
        return Ct(out, t - 2, a.scale * b.scale / self.qq(t))

    def mul_many(self, pairs, twice=False):
        """[mul(a, b, twice) for (a, b) in pairs]: pairs whose products land on one top as batched products (up to
        ops.kmax per call) when the operations have mul_list; the same words"""
        tops = {min(a.top, b.top) for a, b in pairs}
        if len(pairs) == 1 or len(tops) != 1 or not hasattr(self.ops, "mul_list"):
            return [self.mul(a, b, twice) for a, b in pairs]
        t = tops.pop()
        kmax = max(1, getattr(self.ops, "kmax", 1))
        out = []
        for j0 in range(0, len(pairs), kmax):
            grp = pairs[j0:j0 + kmax]
            buf = self.ops.alloc(len(grp))
            self.ops.mul_list(buf, [a.h for a, _ in grp], [b.h for _, b in grp], t, twice)
            out += [Ct(self.ops.item(buf, j), t - 2, a.scale * b.scale / self.qq(t)) for j, (a, b) in enumerate(grp)]
        return out

    def mul_sums(self, groups, adds=None, twice=False):
        """[sum of a b over the pairs (a, b) of g (doubled with twice), plus adds[j] for g = groups[j]], each sum
        relinearized and rescaled once (the operations' mul_sum_list): every pair of every group at one top t, the
        pairs of a group at one product scale, and an addend (None: none; a Ct; or (Ct, k, sub): k times it, subtracted
        with sub) whose multiple sits at that scale, at top t or above, so that it is rescaled with the products.
        Groups go up to ops.kmax per call and up to ops.sum_pairs pairs per call."""
        tops = {min(a.top, b.top) for g in groups for a, b in g}
        assert len(tops) == 1, tops
        t = tops.pop()
        adds = [None] * len(groups) if adds is None else adds
        assert len(adds) == len(groups)
        adds = [None if y is None else y if isinstance(y, tuple) else (y, None, False) for y in adds]
        scales = []
        for g, y in zip(groups, adds):
            s0 = g[0][0].scale * g[0][1].scale
            assert all(abs(a.scale * b.scale / s0 - 1.0) < 1e-9 for a, b in g), [a.scale * b.scale for a, b in g]
            if y is not None:
                ys = y[0].scale * (1 if y[1] is None else y[1])
                assert y[0].top >= t and abs(ys / s0 - 1.0) < 1e-9, (y[0].top, ys, t, s0)
            scales.append(s0 / self.qq(t))
        kmax = max(1, getattr(self.ops, "kmax", 1))
        pmax = max(1, getattr(self.ops, "sum_pairs", 8))
        out, j0 = [], 0
        while j0 < len(groups):
            j1, npairs = j0, 0
            while j1 < len(groups) and j1 - j0 < kmax and npairs + len(groups[j1]) <= pmax:
                npairs += len(groups[j1])
                j1 += 1
            assert j1 > j0, "a group with more pairs than one call takes"
            buf = self.ops.alloc(j1 - j0)
            ys = adds[j0:j1]
            gh = [[(a.h, b.h) for a, b in g] for g in groups[j0:j1]]
            if all(y is None for y in ys) and not twice:
                self.ops.mul_sum_list(buf, gh, t)
            else:
                self.ops.mul_sum_list(buf, gh, t, [None if y is None else y[0].h for y in ys],
                                      sum(1 << j for j, y in enumerate(ys) if y is not None and y[2]),
                                      [None if y is None else y[1] for y in ys], twice)
            out += [Ct(self.ops.item(buf, j - j0), t - 2, scales[j]) for j in range(j0, j1)]
            j0 = j1
        return out

    def prod_meta(self, a, b):
        """(top, scale) of mul(a, b): the product lands two primes below the lower operand's top"""
        t = min(a.top, b.top)
        return t - 2, a.scale * b.scale / self.qq(t)

    def mul_to_many(self, specs):
        """[mul_to(a, c, scale, top) for each spec]: specs whose sources sit at one top as integer products side by
        side and one batched rescale (up to ops.kmax at once); the same words"""
        tops = {sp[0].top for sp in specs}
        if len(specs) == 1 or len(tops) != 1:
            return [self.mul_to(*sp) for sp in specs]
        at = tops.pop()
        buf = self.ops.alloc(len(specs))
        out = []
        for j, (a, c, scale, top) in enumerate(specs):
            assert a.top - 2 >= top, (a.top, top)
            h = self.ops.item(buf, j)
            self.ops.mul_const(h, a.h, a.top, int(round(c * scale * self.qq(a.top) / a.scale)))
            out.append(Ct(h, top, scale))
        kmax = max(1, getattr(self.ops, "kmax", 1))
        for j0 in range(0, len(specs), kmax):
            h = self.ops.item(buf, j0)
            self.ops.rescale2(h, h, at, min(kmax, len(specs) - j0))
        return out

    def mul_to(self, a, c, scale, top):
        """c a landing exactly at (top, scale): a times the integer round(c scale q_a q_b / a.scale), rescaled"""
        assert a.top - 2 >= top, (a.top, top)
        k = int(round(c * scale * self.qq(a.top) / a.scale))
        out = self.ops.alloc()
        self.ops.mul_const(out, a.h, a.top, k)
        self.ops.rescale2(out, out, a.top)
        return Ct(out, top, scale)

    def lincomb(self, terms, c0, top, scale, rescale=True):
        """c0 + sum c_j a_j landing exactly at (top, scale): each a_j (dropped to top + 2) times the integer
        round(c_j scale q_a q_b / a_j.scale) in one weighted sum with the constant, then one rescale (rescale False:
        the sum before it, at (top + 2, scale q_a q_b))"""
        tc = top + 2
        qq = self.qq(tc)
        for a, _ in terms:
            assert a.top >= tc, (a.top, tc)
        ks = [int(round(c * scale * qq / a.scale)) for a, c in terms]
        out = self.ops.alloc()
        self.ops.wsum(out, [a.h for a, _ in terms], tc, ks, int(round(c0 * scale * qq)))
        if not rescale:
            return Ct(out, tc, scale * qq)
        self.ops.rescale2(out, out, tc)
        return Ct(out, top, scale)

    def lincombs(self, specs, raw=()):
        """lincomb of each (terms, c0, top, scale), up to three of them per weighted-sum launch over one source list
        when the operations have wsum_multi (a source a term does not use weighs 0), the sums landing on one top laid
        out side by side and rescaled together (up to ops.kmax per launch sequence): the same words as one lincomb at
        a time. The specs whose index is in raw are left before their rescale: the weighted sum at (top + 2, scale
        q_{top+2} q_{top+1}), for a product to rescale with itself (mul_sums' addend)"""
        if not hasattr(self.ops, "wsum_multi"):
            return [self.lincomb(*sp, rescale=i not in raw) for i, sp in enumerate(specs)]
        groups = []
        for g0 in range(0, len(specs), 3):
            srcs = []
            for terms, _, _, _ in specs[g0:g0 + 3]:
                for a, _ in terms:
                    if not any(x.h is a.h for x in srcs):
                        srcs.append(a)
            if len(srcs) > 8:
                return [self.lincomb(*sp, rescale=i not in raw) for i, sp in enumerate(specs)]
            groups.append((g0, srcs))
        tcs = [top + 2 for _, _, top, _ in specs]
        # the blocks of one top (rescaled together) hold the specs not in raw; each raw one its own buffer
        keys = [(tc, i in raw) for i, tc in enumerate(tcs)]
        blocks = {k: [self.ops.alloc(keys.count(k)), 0] for k in dict.fromkeys(keys) if not k[1]}
        outs = []
        for k in keys:
            if k[1]:
                outs.append(self.ops.alloc())
                continue
            b = blocks[k]
            outs.append(self.ops.item(b[0], b[1]))
            b[1] += 1
        for g0, srcs in groups:
            ks, k0s = [], []
            for terms, c0, top, scale in specs[g0:g0 + 3]:
                qq = self.qq(top + 2)
                for a, _ in terms:
                    assert a.top >= top + 2, (a.top, top + 2)
                w = {id(a.h): int(round(c * scale * qq / a.scale)) for a, c in terms}
                ks.append([w.get(id(x.h), 0) for x in srcs])
                k0s.append(int(round(c0 * scale * qq)))
            self.ops.wsum_multi(outs[g0:g0 + 3], [x.h for x in srcs], tcs[g0:g0 + 3], ks, k0s)
        kmax = max(1, getattr(self.ops, "kmax", 1))
        for (tc, _), (buf, n) in blocks.items():
            for j0 in range(0, n, kmax):
                h = self.ops.item(buf, j0)
                self.ops.rescale2(h, h, tc, min(kmax, n - j0))
        return [Ct(o, top + 2, scale * self.qq(top + 2)) if i in raw else Ct(o, top, scale)
                for i, (o, (_, _, top, scale)) in enumerate(zip(outs, specs))]

    def add(self, a, b, sub=False):
        assert abs(a.scale / b.scale - 1.0) < 1e-9, (a.scale, b.scale)
        t = min(a.top, b.top)
        out = self.ops.alloc()
        self.ops.add(out, a.h, b.h, t, sub)
        return Ct(out, t, a.scale)

    def add_const(self, a, c):
        """in place: the constant c at a's scale added to every slot"""
        self.ops.add_const(a.h, a.top, int(round(c * a.scale)))
        return a

    def double(self, a):
        out = self.ops.alloc()
        self.ops.add(out, a.h, a.h, a.top, False)
        return Ct(out, a.top, a.scale)


class ChebEval:
    """p(u) = sum_k c_k T_k(u) of degree <= 63 on the ciphertext u: the power basis T_1..T_8, T_16, T_32 with every
    T_{a+b} = 2 T_a T_b - T_{|a-b|} formed at one exact scale, then p split by T_32, T_16, T_8 down to leaves of
    degree < 8, each one weighted sum of its T_k with integer constants chosen for the leaf's target (top, scale) and
    one rescale."""

    BABY, GIANTS = 8, (8, 16, 32)

    def __init__(self, ev, fuse=True, fold_ends=True, fold_corr=True):
        self.ev = ev
        self.fuse = fuse  # the chains of remainders in one relinearization each (eval)
        # with fuse: each chain's last leaf added, unrescaled, into the chain's summed product (rescaled with it)
        self.fold_ends = fold_ends
        # with fuse: the basis's corrections T_{a-b} as integer multiples inside their products' sums (basis)
        self.fold_corr = fold_corr

    # T_k = 2 T_a T_b - T_{a-b}, by rounds of independent products (one batched product per round)
    ROUNDS = (((2, 1, 1),), ((3, 2, 1), (4, 2, 2)), ((5, 3, 2), (6, 3, 3), (7, 4, 3), (8, 4, 4)), ((16, 8, 8),),
              ((32, 16, 16),))

    def basis(self, u):
        """T_1..T_8, T_16, T_32. A round that needs corrections T_{a-b} brought to its products' (top, scale) forms
        them together with every later round's whose products' (top, scale) are already known (they follow from the
        operands' alone): one batched rescale for T_3's, T_5's and T_7's"""
        ev = self.ev
        T, corr = {1: u}, {}
        if self.fuse and self.fold_corr and hasattr(ev.ops, "mul_sum_list"):
            # T_k = 2 T_a T_b - T_{a-b}: the correction, times the integer that puts it at the product's scale, is
            # subtracted inside the doubled product's tensor and rescaled with it
            for rnd in self.ROUNDS:
                for t in dict.fromkeys(min(T[a].top, T[b].top) for _, a, b in rnd):
                    sub_r = [(k, a, b) for k, a, b in rnd if min(T[a].top, T[b].top) == t]
                    adds = [None if a == b else (T[a - b], int(round(T[a].scale * T[b].scale / T[a - b].scale)), True)
                            for _, a, b in sub_r]
                    P = ev.mul_sums([[(T[a], T[b])] for _, a, b in sub_r], adds, twice=True)
                    for (k, a, b), p in zip(sub_r, P):
                        T[k] = ev.add_const(p, -1.0) if a == b else p
            self.T = T
            return T
        for i, rnd in enumerate(self.ROUNDS):
            P = dict(zip([k for k, _, _ in rnd], ev.mul_many([(T[a], T[b]) for _, a, b in rnd], twice=True)))
            known = {**T, **P}
            if any(a != b and k not in corr for k, a, b in rnd):
                todo = [(k, a, b) for r in self.ROUNDS[i:] for k, a, b in r
                        if a != b and k not in corr and a in known and b in known]
                specs = []
                for k, a, b in todo:
                    top, scale = ev.prod_meta(known[a], known[b])
                    specs.append((T[a - b], 1.0, scale, top))
                corr.update(zip([k for k, _, _ in todo], ev.mul_to_many(specs)))
            for k, a, b in rnd:
                T[k] = ev.add_const(P[k], -1.0) if a == b else ev.add(P[k], corr[k], sub=True)
        self.T = T
        return T

    def out_top(self):
        """the top the series lands on: the leaves need a product below T_7's top, and three giant products follow"""
        return self.T[7].top - 2 - 6

    def _walk(self, c, top, scale, leaf):
        """the split recursion: leaf(terms, c0, top, scale) for a leaf, else the split [T_g at top + 2, Q, R] (the
        value Q T_g + R) with Q and R walked first"""
        c = np.trim_zeros(np.asarray(c, np.float64), "b")
        ev, T = self.ev, self.T
        if len(c) <= self.BABY:
            terms = [(T[k], float(c[k])) for k in range(1, len(c)) if c[k] != 0.0]
            assert terms, "a leaf with no term of degree >= 1"
            return leaf(terms, float(c[0]), top, scale)
        g = max(x for x in self.GIANTS if x < len(c))
        q, r = cheb_split(c, g)
        G = T[g]
        assert G.top >= top + 2
        Q = self._walk(q, top + 2, scale * ev.qq(top + 2) / G.scale, leaf)
        R = self._walk(r, top, scale, leaf)
        return [Ct(G.h, top + 2, G.scale), Q, R]

    @staticmethod
    def _chain(n):
        """a split's products and its last remainder: Q T_g + R with R = Q' T_g' + R' ... down to a leaf, as the pairs
        [(Q, T_g), (Q', T_g'), ...] and that leaf. Every pair lands on the split's (top, scale): R is walked at the
        split's own (top, scale), and a split's product sits two primes above it at scale times their product"""
        pairs, r = [(n[1], n[0])], n[2]
        while not isinstance(r, Ct):
            pairs.append((r[1], r[0]))
            r = r[2]
        return pairs, r

    def eval(self, c, top, scale):
        """every leaf first (their weighted sums grouped over the shared T_k), then the splits round by round: each
        round's splits whose Q and R are formed take their products Q T_g together where they land on one top. With
        the operations' mul_sum_list, a split whose remainder R is itself a split takes R's products into its own sum
        (one relinearization and rescale for the chain of remainders, their tensors summed); only the root and the
        splits that are some split's Q are formed on their own"""
        specs = []

        def spec(*sp):
            specs.append(sp)
            return len(specs) - 1

        shape = self._walk(c, top, scale, spec)
        fused = self.fuse and hasattr(self.ev.ops, "mul_sum_list")
        # fused: the leaf that ends each chain of remainders stays unrescaled, the chain's addend
        raw = self._chain_ends(shape) if fused and self.fold_ends else set()
        vals = self.ev.lincombs(specs, raw)
        it = iter(vals)
        tree = self._walk(c, top, scale, lambda *sp: next(it))
        if fused:
            return self._eval_chains(tree, {id(vals[i]) for i in raw})
        while not isinstance(tree, Ct):
            ready = []

            def visit(n):
                if isinstance(n, Ct):
                    return
                if isinstance(n[1], Ct) and isinstance(n[2], Ct):
                    ready.append(n)
                else:
                    visit(n[1])
                    visit(n[2])

            visit(tree)
            for t in dict.fromkeys(n[0].top for n in ready):
                grp = [n for n in ready if n[0].top == t]
                for n, P in zip(grp, self.ev.mul_many([(n[1], n[0]) for n in grp])):
                    n.append(self.ev.add(P, n[2]))
            tree = self._resolve(tree)
        return tree

    @staticmethod
    def _chain_ends(n):
        """the leaves (walk indices) that end a chain of remainders: the root's chain's and each chain's whose head is
        some split's Q"""
        ends = set()

        def head(x):
            # x a split: its chain is x, x's R, R's R ... down to a leaf; every Q on the way that is a split heads a
            # chain of its own (a Q that is a leaf is a product's operand)
            while isinstance(x, list):
                if isinstance(x[1], list):
                    head(x[1])
                x = x[2]
            ends.add(x)

        if isinstance(n, list):
            head(n)
        return ends

    def _eval_chains(self, tree, raw=frozenset()):
        """raw: ids of the unrescaled chain-end leaves, each added into its chain's summed product (mul_sums' addend)
        instead of after it"""
        while not isinstance(tree, Ct):
            ready = []

            def visit(n):
                pairs, leaf = self._chain(n)
                if all(isinstance(q, Ct) for q, _ in pairs):
                    ready.append((n, pairs, leaf))
                else:
                    for q, _ in pairs:
                        if not isinstance(q, Ct):
                            visit(q)

            visit(tree)
            for t in dict.fromkeys(min(pairs[0][0].top, pairs[0][1].top) for _, pairs, _ in ready):
                grp = [r for r in ready if min(r[1][0][0].top, r[1][0][1].top) == t]
                adds = [leaf if id(leaf) in raw else None for _, _, leaf in grp]
                for (n, _, leaf), y, P in zip(grp, adds, self.ev.mul_sums([pairs for _, pairs, _ in grp], adds)):
                    n.append(P if y is not None else self.ev.add(P, leaf))
            tree = self._resolve(tree)
        return tree

    @staticmethod
    def _resolve(n):
        """a split whose sum is formed (its fourth entry) becomes that value"""
        if isinstance(n, Ct):
            return n
        if len(n) == 4:
            return n[3]
        n[1], n[2] = ChebEval._resolve(n[1]), ChebEval._resolve(n[2])
        return n


# ----------------------------------------------------------------------------------------------- the composite


class Bootstrap:
    """ModRaise -> CtS (par.budget[0] stages) -> EvalMod (real and imaginary parts) -> StC (par.budget[1] stages) on
    an operations object, with the reference's constants: the collapsed-FFT factors in FIDESlib's layout (lt_plans)
    and the K = 32 EvalMod series with its double angles (EvalModPlan). `primes`: the chain's Q primes (q0 = primes[0], the input's only limb); the input's message
    scale par.delta_in. Plaintexts (the levels' diagonals, the i monomial) are encoded once by `prepare`."""

    def __init__(self, ops, par, primes, ops2=None, special=None, pair=None, fuse_stc=True):
        self.ops, self.par, self.ops2 = ops, par, ops2
        # pair: the two EvalMod chains batched (K = 2) on ops, which must take two ciphertexts per product; by default
        # whenever ops can and no second lane is given
        can = getattr(getattr(ops, "ctx", None), "k_max", 1) >= 2
        self.pair = (ops2 is None and can) if pair is None else bool(pair)
        assert not (self.pair and (ops2 is not None or not can)), "pairing needs one lane on a k_max >= 2 context"
        self.q = [int(p) for p in primes]
        # special primes given: the levels' babies run fused in the extended basis (cts: one ModUp, the products of
        # the key-switched babies before any ModDown, one ModDown per giant step), the diagonals encoded over Q and P
        self.p = None if special is None else [int(x) for x in special]
        self.T = len(self.q) - 1
        self.cts, self.stc, cts_gain = lt_plans(par.N, par.budget)
        # per level (CtS, then StC): fused in the extended basis, else hoisted babies and the plaintext dot over Q. The
        # fused form takes a ModDown per giant step instead of one per baby, so it pays where a level has fewer giant
        # steps than babies (CtS); fuse_stc False keeps the StC levels hoisted
        fz = self.p is not None
        self.fuse = [fz] * len(self.cts) + [fz and fuse_stc] * len(self.stc)
        self.em = EvalModPlan()
        self.ev = Evaluator(ops, self.q)
        self.q0 = float(self.q[0])
        # CtS: the raised ciphertext (P = m + q0 I) is first multiplied by the integer c = 2^e that lifts 2 q0 K near
        # par.target: the baby rotations' key-switch noise is added to integers that large, not to the raw P (about
        # 2 q0 K). Its label carries 2 q0 K c times the CtS stages' gain n (OpenFHE's unnormalised inverse), so that
        # after the stages the values are brev(U0^-1 decode(P)) / (2 q0 K), the EvalMod input; each stage multiplies
        # the label by f so that this input sits at par.target exactly (the reference rides the same 1 / (K n) on its
        # post-raise constant, crates/pc-gpu/src/bts/dense.rs)
        self.lift = 1 << max(0, int(math.floor(math.log2(par.target / (2.0 * self.q0 * par.K)))))
        self.raise_scale = 2.0 * self.q0 * par.K * self.lift * cts_gain
        self.cts_f = (par.target / self.raise_scale) ** (1.0 / len(self.cts))
        self.top_out = self.T - 2 * (len(self.cts) + 7 + par.r + len(self.stc))
        assert self.top_out >= 0, "the chain is too short for the bootstrap"

    def steps(self):
        """every rotation step the linear transforms take"""
        out = []
        for p in self.cts + self.stc:
            for s in p.steps():
                if s not in out:
                    out.append(s)
        return out

    def prepare(self):
        """encode every level's diagonals (at the level's input top, scale q_a q_b f) and the i monomial"""
        ops, N = self.ops, self.par.N
        self.pts, self.pt_s = [], []
        top = self.T
        for plans, f in ((self.cts, self.cts_f), (self.stc, 1.0)):
            for p in plans:
                fused = self.fuse[len(self.pts)]
                sc = self.ev.qq(top) * f
                prim = self.q[: top + 1] + (self.p if fused else [])
                coef = [[None if d is None else encode_rows(d, N, sc, prim) for d in p.pts[j]] for j in range(p.G)]
                # the plaintext dot (and the fused stage) reads a level's diagonals at one compact width
                s = min((compact_shift(c) for r in coef for c in r if c is not None), default=0)
                row = []
                for j in range(p.G):
                    for i in range(p.B):
                        c = coef[j][i]
                        if c is None:
                            row.append(None)
                        elif not fused:
                            row.append(ops.plaintext(c, top, s))
                        else:
                            row.append(ops.plaintext_ext(c, top, s))
                self.pts.append(row)
                self.pt_s.append(s)
                top -= 2
                if plans is self.cts and p is self.cts[-1]:
                    top -= 2 * (7 + self.par.r)
        mono = np.zeros((len(self.q), N), np.uint32)
        mono[:, N // 2] = 1  # X^(N/2): i in every slot
        self.mono_i = ops.plaintext(mono, self.T)
        mono_m = np.zeros((len(self.q), N), np.uint32)
        mono_m[:, N // 2] = [p - 1 for p in self.q]  # -X^(N/2): -i
        self.mono_mi = ops.plaintext(mono_m, self.T)

    def lt(self, x, plan, pts, f, s=0, rots=None, dest=None, fused=False):
        """one BSGS level: pts its diagonals (None where zero), s their compact shift (rows of width N >> s). rots: a
        buffer of B ciphertexts whose first already holds x (else x is copied into a new one); dest: where the output
        goes (else a new ciphertext); fused: the babies in the extended basis (pts encoded over Q and P)"""
        ops, top = self.ops, x.top
        B, G = plan.B, plan.G
        res = ops.alloc(G)
        if not fused:
            if rots is None:
                rots = ops.alloc(B)
                ops.copy(ops.item(rots, 0), x.h, top)
            ops.hoisted(ops.item(rots, 1), x.h, top, [b % self.par.n for b in plan.baby[1:]])
            ops.pt_dot(res, rots, top, pts, B, G, s)
        else:
            ops.cts(res, x.h, top, pts, B, G, s)
        # the giant steps: the rotated results' key dots summed in the extended basis, one ModDown onto the
        # unrotated result
        if fused:
            # the fused stage's G extended results brought down to Q, one batched ModDown where the operations have it
            q = ops.alloc(G)
            if hasattr(ops, "moddown_k"):
                ops.moddown_k(q, res, top, G)
            else:
                for j in range(G):
                    ops.moddown(ops.item(q, j), ops.item(res, j), top)
            res = q
        base, ys, gs = None, [], []
        for j in range(G):
            g = plan.giant[j] % self.par.n
            y = ops.item(res, j)
            if g:
                ys.append(y)
                gs.append(g)
            elif base is None:
                base = y
            else:
                t = ops.alloc()
                ops.add(t, base, y, top, False)
                base = t
        out = ops.alloc() if dest is None else dest
        if ys:
            # the rescale by the two top primes fused into the sum's ModDown
            ops.rotate_many_rescale(out, ys, top, gs, base)
        else:
            ops.rescale2(out, base, top)
        ops.level_done()
        return Ct(out, top - 2, x.scale * f)

    def evalmod(self, u, ev=None):
        ev = ev or self.ev
        ce = ChebEval(ev)
        ce.basis(u)
        top = ce.out_top()
        h = ce.eval(self.em.c, top, ev.qq(top))
        for sc in self.em.scalars:
            h = ev.add_const(ev.mul(h, h, twice=True), sc)
        return h

    def run(self, x_h):
        """x_h: the input ciphertext at top 0 (message scale par.delta_in). Returns the output Ct (its top and scale:
        slot values = the input's message)."""
        ops, ev, par = self.ops, self.ev, self.par
        ops.begin()
        if self.ops2 is not None:
            self.ops2.begin()
        # each level's input is written straight into the first slot of that level's rotation buffer (the plaintext
        # dot reads the unrotated input there), so no level copies it
        plans = self.cts + self.stc
        hoist = [not fz for fz in self.fuse]
        nxt = ops.alloc(plans[0].B) if hoist[0] else None
        raised = ops.item(nxt, 0) if hoist[0] else ops.alloc()
        ops.mod_raise(raised, x_h, self.T)
        ops.mul_const(raised, raised, self.T, self.lift)
        x = Ct(raised, self.T, self.raise_scale)
        k = 0
        for i, p in enumerate(self.cts):
            rots = nxt
            nxt = ops.alloc(plans[k + 1].B) if hoist[k + 1] and i + 1 < len(self.cts) else None
            x = self.lt(x, p, self.pts[k], self.cts_f, self.pt_s[k], rots=rots,
                        dest=ops.item(nxt, 0) if nxt is not None else None, fused=self.fuse[k])
            k += 1
        cj = ops.alloc()
        ops.rotate(cj, x.h, x.top, "conj")
        pair = ops.alloc(2) if self.pair else None
        re = Ct(ops.item(pair, 0) if self.pair else ops.alloc(), x.top, x.scale)
        ops.add(re.h, x.h, cj, x.top, False)
        d = ops.alloc()
        ops.add(d, x.h, cj, x.top, True)
        im = Ct(ops.item(pair, 1) if self.pair else ops.alloc(), x.top, x.scale)
        ops.mul_pt(im.h, d, x.top, self.mono_mi)
        if self.pair:
            # both chains in the same launches: the pair's ciphertext 0 is the real part's, 1 the imaginary part's
            h = self.evalmod(Ct(pair, x.top, x.scale), Evaluator(PairOps(ops), self.q))
            re, im = Ct(ops.item(h.h, 0), h.top, h.scale), Ct(ops.item(h.h, 1), h.top, h.scale)
        elif self.ops2 is None:
            re, im = self.evalmod(re), self.evalmod(im)
        else:
            # the imaginary part's chain on the second lane (its own workspace and stream), beside the real part's
            ops.fork(self.ops2)
            im = self.evalmod(im, Evaluator(self.ops2, self.q))
            re = self.evalmod(re)
            ops.join(self.ops2)
        ii = ops.alloc()
        ops.mul_pt(ii, im.h, im.top, self.mono_i)
        nxt = ops.alloc(self.stc[0].B) if hoist[k] else None
        if hoist[k]:
            assert abs(re.scale / im.scale - 1.0) < 1e-9 and re.top == im.top
            ops.add(ops.item(nxt, 0), re.h, ii, re.top, False)
            w = Ct(ops.item(nxt, 0), re.top, re.scale)
        else:
            w = ev.add(re, Ct(ii, im.top, im.scale))
        for i, p in enumerate(self.stc):
            rots = nxt
            nxt = ops.alloc(plans[k + 1].B) if i + 1 < len(self.stc) and hoist[k + 1] else None
            w = self.lt(w, p, self.pts[k], 1.0, self.pt_s[k], rots=rots,
                        dest=ops.item(nxt, 0) if nxt is not None else None, fused=self.fuse[k])
            k += 1
        # the slot values are now sin(2 pi P / q0) / (2 pi) ~ m / q0: 1 / q0 times the message's at the input's
        # scale: relabel
        w.scale = w.scale * par.delta_in / self.q0
        return w

    def precision_bits(self, err):
        return -math.log2(err) if err > 0 else float("inf")


# ----------------------------------------------------------------------------------------------- device operations


class View:
    """A ciphertext inside a device buffer (word offset), addressable like a DevBuf by the engine's calls."""
    __slots__ = ("buf", "off")

    def __init__(self, buf, off=0):
        self.buf, self.off = buf, off

    def addr(self, offset=0):
        return self.buf.addr(self.off + offset)


def key_plan(boot):
    """The galois elements of the bootstrap's key group, one slot per use: per linear-transform level its babies
    (consecutive, so that the hoisted rotations batch their ModDowns) then its giants; the conjugation last. Returns
    (galois list, per level (baby key indices, {giant step: key index}), conj index)."""
    N, n = boot.par.N, boot.par.n
    gal, levels = [], []
    for p in boot.cts + boot.stc:
        babies = []
        for b in p.baby[1:]:
            babies.append(len(gal))
            gal.append(pow(5, b % n, 2 * N))
        giants = {}
        for g in p.giant:
            g %= n
            if g and g not in giants:
                giants[g] = len(gal)
                gal.append(pow(5, g, 2 * N))
        levels.append((babies, giants))
    gal.append(2 * N - 1)
    return gal, levels, len(gal) - 1


class PairOps:
    """The real and imaginary parts' EvalMod chains side by side: every handle is two consecutive ciphertexts of one
    GpuOps buffer, every operation one launch sequence for both (K = 2). Both chains take the same steps with the same
    constants, so each part's words are those of its chain run alone."""

    def __init__(self, ops):
        self.o = ops
        self.kmax = max(1, ops.kmax // 2)

    def alloc(self, count=1):
        return self.o.alloc(2 * count)

    def item(self, h, i):
        return self.o.item(h, 2 * i)

    def add(self, out, a, b, top, sub):
        self.o.add(out, a, b, top, sub, K=2)

    def mul_const(self, out, x, top, k):
        self.o.mul_const(out, x, top, k, K=2)

    def add_const(self, x, top, k):
        self.o.add_const(x, top, k, K=2)

    def wsum(self, out, srcs, top, ks, k0):
        self.o.wsum(out, srcs, top, ks, k0, K=2)

    def wsum_multi(self, outs, srcs, tops, ks, k0s):
        self.o.wsum_multi(outs, srcs, tops, ks, k0s, K=2)

    def mul_relin_rescale(self, out, a, b, top, twice=False):
        self.o.mul_relin_rescale(out, a, b, top, K=2, twice=twice)

    def rescale2(self, out, x, top, count=1):
        self.o.rescale2(out, x, top, K=2 * count)

    def mul_list(self, out, a, b, top, twice=False):
        ex = lambda hs: [self.o.item(h, i) for h in hs for i in (0, 1)]
        self.o.mul_list(out, ex(a), ex(b), top, twice)

    @property
    def sum_pairs(self):
        return max(1, getattr(self.o, "sum_pairs", 8) // 2)

    def mul_sum_list(self, out, groups, top, adds=None, sub=0, kmuls=None, twice=False):
        ys = None if adds is None else [None if y is None else self.o.item(y, i) for y in adds for i in (0, 1)]
        sub2 = sum(3 << 2 * j for j in range(len(groups)) if (sub >> j) & 1)
        ks = None if kmuls is None else [k for k in kmuls for _ in (0, 1)]
        self.o.mul_sum_list(out, [[(self.o.item(a, i), self.o.item(b, i)) for a, b in g] for g in groups
                                  for i in (0, 1)], top, ys, sub2, ks, twice)


class GpuOps:
    """The composite's operations on the device: the engine's key switches, rescale and products, the kernel table's
    element-wise entries (ew_add, ew_scale, ew_copy, add_const, mul_table, pt_dot, mod_raise). Buffers come from a
    pool reused in request order (begin() rewinds it), constants and plaintexts are cached on the device, so that a
    second run allocates nothing."""

    def __init__(self, ctx, keys, relin, levels, conj, stream):
        from . import abi, bts, engine
        from ._lib import LIB

        self.abi, self.eng, self.LIB = abi, engine, LIB
        self.ctx, self.keys, self.relin, self.st = ctx, keys, relin, stream
        self.levels, self.conj_key = levels, conj
        self.N, self.R, self.nq = ctx.n, ctx.rows, ctx.nq
        self.cw = ctx.ct_words
        self.kmax = ctx.k_max  # ciphertexts per batched rescale
        # the fused stage's words by the hoisted route (babies' keys regenerated once per level) instead of cts_k
        self.cts_hoisted = True
        self.primes = [int(p) for p in ctx.chain.primes]
        self.pr = LIB.pcx_ctx_primes(ctx.h)
        self.pool, self.cur = [], 0
        self.cache = {}
        self.level_i = 0
        self.zero_pt = None
        self.mr_consts = bts.mod_raise_consts(self.primes, 1)
        self.lvl_of_plan = {}

    # -- buffers
    def begin(self):
        self.cur = 0
        self.level_i = 0

    def alloc(self, count=1):
        if self.cur < len(self.pool) and self.pool[self.cur][1] == count:
            buf = self.pool[self.cur][0]
        else:
            buf = self.eng.DevBuf(count * self.cw)
            if self.cur < len(self.pool):
                self.pool[self.cur] = (buf, count)
            else:
                self.pool.append((buf, count))
        self.cur += 1
        return View(buf, 0)

    def item(self, h, i):
        return View(h.buf, h.off + i * self.cw)

    def _ref(self, h):
        return self.abi.PolyRef(h.addr().value, self.cw, self.R * self.N)

    def _call(self, name, a):
        rc = self.abi.call(name, a, self.st, self.ctx.logn)
        if rc != 0:
            raise self.eng.HipError(f"{name} returned {rc}")

    def _ew(self, name, out, a, b, top, sub=0, sc=None, K=1):
        e = self.abi.EwArgs()
        e.out, e.a = self._ref(out), self._ref(a)
        if b is not None:
            e.b = self._ref(b)
        e.rs = self.abi.RowSet(top + 1, 0, self.nq, 0)
        if sc is not None:
            e.sc, e.scs = sc[0].ptr.value, sc[1].ptr.value
        e.pr, e.K, e.nparts, e.sub = self.pr, K, 2, sub
        self._call(name, e)

    # -- element-wise
    def copy(self, dst, src, top):
        self._ew("ew_copy", dst, src, None, top)

    def add(self, out, a, b, top, sub, K=1):
        self._ew("ew_add", out, a, b, top, 1 if sub else 0, K=K)

    def _const_rows(self, k):
        key = ("k", k)
        if key not in self.cache:
            r = np.array([k % p for p in self.primes], np.uint32)
            rs = np.array([(int(v) << 32) // p for v, p in zip(r, self.primes)], np.uint64).astype(np.uint32)
            self.cache[key] = (self.eng.DevBuf.from_array(r), self.eng.DevBuf.from_array(rs))
        return self.cache[key]

    def mul_const(self, out, x, top, k, K=1):
        self._ew("ew_scale", out, x, None, top, sc=self._const_rows(int(k)), K=K)

    def add_const(self, x, top, k, K=1):
        r, _ = self._const_rows(int(k))
        a = self.abi.AddConstArgs()
        a.x, a.k, a.pr, a.n, a.K = self._ref(x), r.ptr.value, self.pr, top + 1, K
        self._call("add_const", a)

    def wsum(self, out, srcs, top, ks, k0, K=1):
        key = ("w", tuple(ks), k0)
        if key not in self.cache:
            w = np.array([[k % p for p in self.primes] for k in ks], np.uint32)
            ws = np.array([[(int(v) << 32) // p for v, p in zip(r, self.primes)] for r in w], np.uint64)
            kr = np.array([k0 % p for p in self.primes], np.uint32)
            self.cache[key] = tuple(self.eng.DevBuf.from_array(v) for v in (w, ws.astype(np.uint32), kr))
        bw, bws, bk = self.cache[key]
        a = self.abi.WsumKArgs()
        a.w.out = self._ref(out)
        for j, x in enumerate(srcs):
            a.w.src[j] = self._ref(x)
        a.w.w, a.w.ws, a.w.pr = bw.ptr.value, bws.ptr.value, self.pr
        a.w.nsrc, a.w.rowstride, a.w.n, a.w.K = len(srcs), self.R, top + 1, K
        a.k = bk.ptr.value
        self._call("wsum_k", a)

    def wsum_multi(self, outs, srcs, tops, ks, k0s, K=1):
        """up to 3 weighted sums of one source list in one launch (the table's wsum_multi): outs[m] = sum_j ks[m][j]
        srcs[j] + k0s[m] on rows 0..tops[m]"""
        key = ("wm", tuple(tuple(k) for k in ks), tuple(k0s))
        if key not in self.cache:
            bufs = []
            for km, k0 in zip(ks, k0s):
                w = np.array([[k % p for p in self.primes] for k in km], np.uint32)
                ws = np.array([[(int(v) << 32) // p for v, p in zip(r, self.primes)] for r in w], np.uint64)
                kr = np.array([k0 % p for p in self.primes], np.uint32)
                bufs.append(tuple(self.eng.DevBuf.from_array(v) for v in (w, ws.astype(np.uint32), kr)))
            self.cache[key] = bufs
        bufs = self.cache[key]
        a = self.abi.WsumMultiArgs()
        for m, o in enumerate(outs):
            a.out[m] = self._ref(o)
            a.w[m], a.ws[m], a.k[m] = (b.ptr.value for b in bufs[m])
            a.n[m] = tops[m] + 1
        for j, x in enumerate(srcs):
            a.src[j] = self._ref(x)
        a.pr, a.nout, a.nsrc, a.rowstride, a.K = self.pr, len(outs), len(srcs), self.R, K
        a.nmax = max(t + 1 for t in tops)
        self._call("wsum_multi", a)

    def mul_pt(self, out, x, top, pt):
        a = self.abi.MulTableArgs()
        a.out, a.in_, a.t, a.pr, a.n, a.K = self._ref(out), self._ref(x), pt.ptr.value, self.pr, top + 1, 1
        self._call("mul_table", a)

    # -- plaintexts
    def _rows(self, roff, ids):
        key = ("rows", tuple(roff), tuple(ids))
        if key not in self.cache:
            self.cache[key] = self.eng.Rows(self.ctx, roff, ids)
        return self.cache[key]

    def plaintext(self, coef_rows, top, s=0):
        """coefficient residue rows 0..top -> a device plaintext [top + 1][N] in evaluation form; with s > 0 (a
        polynomial in X^(2^s)) its compact form [top + 1][N >> s], one word per block of 2^s equal ones"""
        buf = self.eng.DevBuf.from_array(np.ascontiguousarray(coef_rows[: top + 1], np.uint32))
        self._rows(list(range(top + 1)), list(range(top + 1))).ntt(buf, 1, self.st)
        self.st.sync()
        if s:
            buf = self.eng.DevBuf.from_array(compact_rows(buf.download((top + 1, self.N), self.st), s))
        return buf

    def plaintext_ext(self, coef_rows, top, s=0):
        """coefficient residue rows over Q 0..top then the special primes -> a device plaintext [top + 1 + kp][N] in
        evaluation form (the extended basis of the fused stage); compact [top + 1 + kp][N >> s] as plaintext's"""
        kp = self.R - self.nq
        rows = top + 1 + kp
        buf = self.eng.DevBuf.from_array(np.ascontiguousarray(coef_rows[:rows], np.uint32))
        ids = list(range(top + 1)) + [self.nq + j for j in range(kp)]
        self._rows(list(range(rows)), ids).ntt(buf, 1, self.st)
        self.st.sync()
        if s:
            buf = self.eng.DevBuf.from_array(compact_rows(buf.download((rows, self.N), self.st), s))
        return buf

    def cts(self, res, x, top, pts, B, G, s=0):
        """res_j = sum_i rot_i(x) pt_{B j + i} in the extended basis (pcx_cts_stage: one ModUp, the babies' key
        switches before ModDown, keys regenerated in the kernel; or its hoisted route); s: the diagonals' compact
        shift"""
        ptw, enc = self.N >> s, (0x7F000000 | s) if s else 0xFFFFFFFF
        key = ("cptr", tuple(id(p) for p in pts))
        if key not in self.cache:
            if any(p is None for p in pts) and "zero_ext" not in self.cache:
                z = self.eng.DevBuf(self.R * self.N)
                z.zero()
                self.cache["zero_ext"] = z
            ptrs = np.array([(self.cache["zero_ext"] if p is None else p).ptr.value for p in pts], np.uint64)
            self.cache[key] = self.eng.DevBuf.from_array(ptrs.view(np.uint32))
        babies = self.levels[self.level_i][0]
        if self.cts_hoisted:
            rot = self.alloc(B)
            self.ctx.cts_stage_hoisted(self.keys, babies[0] if babies else 0, B, G, self.cache[key], B * G, ptw, enc,
                                       x, top, rot, res, self.st)
        else:
            self.ctx.cts_stage(self.keys, babies[0] if babies else 0, B, G, self.cache[key], B * G, ptw, enc, x, top,
                               res, self.st)

    def moddown_k(self, out, ext, top, m):
        self.ctx.moddown_k(ext, top, out, m, self.st)

    def moddown(self, out, ext, top):
        self.ctx.moddown(ext, top, out, self.st)

    def pt_dot(self, res, rots, top, pts, B, G, s=0):
        key = ("ptr", tuple(id(p) for p in pts))
        if key not in self.cache:
            if any(p is None for p in pts) and self.zero_pt is None:
                self.zero_pt = self.eng.DevBuf((self.nq) * self.N)
                self.zero_pt.zero()
            ptrs = np.array([(self.zero_pt if p is None else p).ptr.value for p in pts], np.uint64)
            self.cache[key] = self.eng.DevBuf.from_array(ptrs.view(np.uint32))
        a = self.abi.PtDotArgs()
        a.rot = self.abi.PolyRef(rots.addr().value, B * self.cw, self.R * self.N)
        a.res = self.abi.PolyRef(res.addr().value, G * self.cw, self.R * self.N)
        a.rot_stride, a.res_stride = self.cw, self.cw
        a.pts, a.pr = self.cache[key].ptr.value, self.pr
        a.rs = self.abi.RowSet(top + 1, 0, self.nq, 0)
        a.npts, a.bstep, a.gstep, a.K, a.pt_prow = B * G, B, G, 1, top + 1
        # compact diagonals: word i of a row read at i >> s (a zero diagonal reads the full-width zero rows)
        a.ptw, a.enc = self.N >> s, (0x7F000000 | s) if s else 0xFFFFFFFF
        self._call("pt_dot", a)

    # -- key switches
    def rotate(self, out, x, top, step):
        if step == "conj":
            r = self.conj_key
        else:
            r = self.levels[self.level_i][1][step]
        self.ctx.rotate(self.keys, r, x, top, out, self.st)

    def rotate_many(self, out, xs, top, steps, onto):
        r = [self.levels[self.level_i][1][g] for g in steps]
        self.ctx.rotate_many(self.keys, r, xs, top, out, self.st, onto=onto)

    def rotate_many_rescale(self, out, xs, top, steps, onto):
        r = [self.levels[self.level_i][1][g] for g in steps]
        self.ctx.rotate_many_rescale(self.keys, r, xs, top, out, self.st, onto=onto)

    def hoisted(self, outs, x, top, steps):
        babies = self.levels[self.level_i][0]
        assert len(babies) == len(steps)
        self.ctx.rotate_hoisted(self.keys, babies, x, top, outs, self.st)

    def level_done(self):
        self.level_i += 1

    def fork(self, other):
        """other's stream waits for the work queued on this one"""
        if "fork" not in self.cache:
            self.cache["fork"] = (self.eng.Event(), self.eng.Event())
        e = self.cache["fork"][0]
        e.record(self.st)
        other.st.wait(e)

    def join(self, other):
        """this stream waits for the work queued on other's"""
        e = self.cache["fork"][1]
        e.record(other.st)
        self.st.wait(e)

    def mul_relin(self, out, a, b, top):
        self.ctx.mul_relin(self.relin, a, b, top, out, self.st)

    def mul_relin_rescale(self, out, a, b, top, twice=False, K=1):
        self.ctx.mul_relin_rescale(self.relin, a, b, top, out, self.st, K=K, twice=twice)

    def rescale2(self, out, x, top, K=1):
        self.ctx.rescale(x, top, 2, out, self.st, K=K)

    def mul_list(self, out, a, b, top, twice=False):
        """out's len(a) consecutive ciphertexts = a[j] b[j], relinearized and rescaled (the pairs at their own
        addresses)"""
        self.ctx.mul_relin_rescale_list(self.relin, a, b, top, out, self.st, twice=twice)

    sum_pairs = 8  # pairs per pcx_mul_sum_relin_rescale_list call

    def mul_sum_list(self, out, groups, top, adds=None, sub=0, kmuls=None, twice=False):
        """out's len(groups) consecutive ciphertexts: product j = the sum of a b over the pairs of groups[j] (doubled
        with twice) plus kmuls[j] adds[j] (None: nothing; a multiplier None: 1; subtracted where bit j of sub is set),
        relinearized and rescaled once"""
        kb = None if kmuls is None else [None if k is None else self._krows(int(k)) for k in kmuls]
        self.ctx.mul_sum_relin_rescale_list(self.relin, groups, top, out, self.st, adds, sub, kb, twice)

    def _krows(self, k):
        """the integer k as device rows: k mod q by prime id, then their Shoup companions (one buffer, cached)"""
        key = ("kr", k)
        if key not in self.cache:
            r = np.array([k % p for p in self.primes], np.uint32)
            rs = np.array([(int(v) << 32) // p for v, p in zip(r, self.primes)], np.uint64).astype(np.uint32)
            self.cache[key] = self.eng.DevBuf.from_array(np.concatenate([r, rs]))
        return self.cache[key]

    # -- ModRaise
    def mod_raise(self, out, x, top):
        self._ew("ew_copy", out, x, None, 0)
        R = self.R
        self._rows([0, R], [0, 0]).ntt(out, -1, self.st)
        qhatinv, qhat = self.mr_consts
        a = self.abi.ModRaiseArgs()
        a.x, a.pr = out.addr().value, self.pr
        a.ct_stride, a.part_stride = self.cw, R * self.N
        for k in range(4):
            a.qhatinv[k] = qhatinv[k]
            for t in range(64):
                a.qhat[k][t] = qhat[k][t]
        a.K, a.d, a.r0, a.r1, a.nparts = 1, 1, 1, top + 1, 2
        self._call("mod_raise", a)
        rows = list(range(top + 1))
        self._rows(rows + [R + t for t in rows], rows + rows).ntt(out, 1, self.st)
