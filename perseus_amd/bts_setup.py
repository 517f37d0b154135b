"""The reference's bootstrap constants, restated on the host: the EvalMod Chebyshev series (crates/pc-core/src/
bts_setup.rs:133-165 cheb_interp, evalmod_k32_low) and OpenFHE's collapsed-FFT CoeffsToSlots / SlotsToCoeffs factors
with their BSGS parameters (bts_setup.rs:245-575 reduce_rotation, select_layers, collapsed_fft_params, rot_group,
ksi_pows, CoeffEncodingOneLevel / CoeffDecodingOneLevel and their collapses, FftStage, cts_stc_factors) in FIDESlib's
"LT-friendly" stage layout (bts_setup.rs:818-940 fides_layout), plus OpenFHE's rotation sets (:722-816).

The values are meant to equal the reference's to the last bit, so every floating-point value is formed by the same
operations in the same order:
- sums run left to right, as Rust's Iterator::sum does; a vectorised sum adds its terms in that order;
- cos / sin / pow are the C library's (Python's math module), as Rust's f64 methods are;
- a complex product is (ac - bd, ad + bc) formed from separate real products (numpy's complex ufuncs may fuse a
  multiply and an add);
- where a vector receives more than two contributions they are added in the reference's loop order.
Complex vectors are numpy complex128 arrays; the products go through `cmul`.
"""
import math

import numpy as np


# ----------------------------------------------------------------------------------------------- complex helpers
def cx(re, im):
    out = np.empty(np.shape(re), np.complex128)
    out.real, out.imag = re, im
    return out


def cmul(a, b):
    """(ac - bd, ad + bc) elementwise, each product and sum rounded on its own"""
    a, b = np.asarray(a, np.complex128), np.asarray(b, np.complex128)
    ar, ai, br, bi = a.real, a.imag, b.real, b.imag
    return cx(ar * br - ai * bi, ar * bi + ai * br)


def cscale(a, s):
    a = np.asarray(a, np.complex128)
    return cx(a.real * s, a.imag * s)


# ----------------------------------------------------------------------------------------------- EvalMod series
def cheb_interp(deg, parity, f):
    """The Chebyshev interpolant of f on [-1, 1] at degree deg, in the evaluator convention (c0 not halved: the
    polynomial is c0 / 2 + sum_{k >= 1} c_k T_k): c_k = (2 / n) sum_j f(cos t_j) cos(k t_j), t_j = pi (j + 1/2) / n,
    n = deg + 1; parity 0 / 1 keeps the even / odd coefficients only, 2 all (bts_setup.rs:133-151)."""
    n = deg + 1
    th = [math.pi * (j + 0.5) / n for j in range(n)]
    fv = [f(math.cos(t)) for t in th]
    out = []
    for k in range(n):
        if parity < 2 and k % 2 != parity:
            out.append(0.0)
            continue
        s = 0.0
        for j in range(n):
            s += fv[j] * math.cos(k * th[j])
        out.append(s * 2.0 / n)
    return out


EVALMOD_K32 = 32.0
EVALMOD_K32_LOW_DEG = 59
EVALMOD_K32_LOW_DA_ITS = 3


def evalmod_k32_low():
    """(2 pi)^(-1/8) cos(2 pi (32 y - 1/4) / 8) at Chebyshev degree 59; after 3 double angles (double_angle_scalar)
    the series reads sin(2 pi 32 y) / (2 pi) (bts_setup.rs:153-165)."""
    r = float(1 << EVALMOD_K32_LOW_DA_ITS)
    pi = math.pi
    pre = (2.0 * pi) ** (-1.0 / r)
    return cheb_interp(EVALMOD_K32_LOW_DEG, 2, lambda y: pre * math.cos(2.0 * pi * (32.0 * y - 0.25) / r))


def double_angle_scalar(j, r):
    """The constant of double-angle step j (1..r) at the shipped output amplitude 1 / (2 pi): x -> 2 x^2 + scalar
    with scalar = -1 / (2 pi)^(2^(j - r)) (crates/pc-shadow/src/evalmod.rs:954-964, OpenFHE's
    ApplyDoubleAngleIterations). A series a cos(t) with a = (2 pi)^(-1 / 2^r) becomes (2 pi)^-1 cos(2^r t)."""
    return -1.0 / (2.0 * math.pi) ** (2.0 ** (j - r))


# ----------------------------------------------------------------------------------------------- collapsed FFT
def reduce_rotation(index, slots):
    """OpenFHE ReduceRotation: for power-of-two slots a negative exact multiple of slots maps to slots, not 0
    (bts_setup.rs:245-256)."""
    if slots & (slots - 1) == 0:
        n = slots.bit_length() - 1
        if index >= 0:
            return index - ((index >> n) << n)
        return index + slots + ((abs(index) >> n) << n)
    return (slots + int(math.fmod(index, slots))) % slots  # Rust's % keeps the dividend's sign


def select_layers(log_slots, budget):
    """OpenFHE SelectLayers -> (layers, rows, rem) (bts_setup.rs:258-279)."""
    layers = math.ceil(log_slots / budget)
    rows = log_slots // layers
    rem = log_slots % layers
    dim = rows + (rem != 0)
    if dim < budget:
        layers -= 1
        rows = log_slots // layers
        rem = log_slots - rows * layers
        dim = rows + (rem != 0)
        if dim > budget:
            while dim != budget:
                rows -= 1
                rem = log_slots - rows * layers
                dim = rows + (rem != 0)
    return layers, rows, rem


class CollapsedFftParams:
    """OpenFHE GetCollapsedFFTParams (bts_setup.rs:283-338): b giant steps, g baby steps."""

    FIELDS = ("level_budget", "layers_collapse", "rem_collapse", "num_rotations", "b", "g", "num_rotations_rem",
              "b_rem", "g_rem")

    def __init__(self, slots, level_budget, dim1):
        if slots == 0 or level_budget == 0:
            raise ValueError(f"collapsed_fft_params: slots={slots} level_budget={level_budget}")
        log_slots = 1 if slots < 3 else slots.bit_length() - 1
        layers, _rows, rem = select_layers(log_slots, level_budget)
        nr = (1 << (layers + 1)) - 1
        nr_rem = (1 << (rem + 1)) - 1
        g = (1 << (layers // 2 + 1 + (nr > 7))) if dim1 == 0 or dim1 > nr else dim1
        self.level_budget, self.layers_collapse, self.rem_collapse = level_budget, layers, rem
        self.num_rotations, self.g, self.b = nr, g, (nr + 1) // g
        self.num_rotations_rem = nr_rem
        self.g_rem = (1 << (rem // 2 + 1 + (nr_rem > 7))) if rem else 0
        self.b_rem = (nr_rem + 1) // self.g_rem if rem else 0

    def astuple(self):
        return tuple(getattr(self, f) for f in self.FIELDS)


def rot_group(slots, m):
    """5^i mod m, i < slots (bts_setup.rs:340-350)"""
    v, f, mask = [], 1, m - 1
    for _ in range(slots):
        v.append(f)
        f = (f * 5) & mask
    return np.array(v, np.int64)


def ksi_pows(m):
    """exp(2 pi i j / m) for j <= m, the last equal to the first (bts_setup.rs:352-358)"""
    ak = 2.0 * math.pi / m
    re = [math.cos(ak * j) for j in range(m)]
    im = [math.sin(ak * j) for j in range(m)]
    v = cx(np.array(re), np.array(im))
    return np.concatenate([v, v[:1]])


_ONE = complex(1.0, 0.0)


def _unit(flag_i, m, sign):
    """the layer's multiplier b: 1, or exp(sign i pi / 2) (cos and sin evaluated, not exact) on the m = 2 layer"""
    if flag_i and m == 2:
        return complex(math.cos(sign * math.pi / 2.0), math.sin(sign * math.pi / 2.0))
    return _ONE


def coeff_encoding_one_level(pows, rg, flag_i):
    """OpenFHE CoeffEncodingOneLevel: 3 log2(slots) vectors (bts_setup.rs:366-399)"""
    dim = len(pows) - 1
    slots = len(rg)
    ls = slots.bit_length() - 1
    coeff = np.zeros((3 * ls, slots), np.complex128)
    m = slots
    k = np.arange(slots)
    while m > 1:
        s0 = m.bit_length() - 2
        s1, s2 = s0 + ls, s0 + 2 * ls
        b = _unit(flag_i, m, -1)
        lenq, lenh = m << 2, m >> 1
        pos = k % m
        first = pos < lenh
        coeff[s2, first] = b
        coeff[s1, first] = b
        j = pos[~first] - lenh
        w = cmul(np.full(j.shape, b), pows[(lenq - rg[j] % lenq) * (dim // lenq)])
        coeff[s1, ~first] = -w
        coeff[s0, ~first] = w
        m >>= 1
    return coeff


def coeff_decoding_one_level(pows, rg, flag_i):
    """OpenFHE CoeffDecodingOneLevel (bts_setup.rs:401-435)"""
    dim = len(pows) - 1
    slots = len(rg)
    ls = slots.bit_length() - 1
    coeff = np.zeros((3 * ls, slots), np.complex128)
    m = 2
    k = np.arange(slots)
    while m <= slots:
        s0 = m.bit_length() - 2
        s1, s2 = s0 + ls, s0 + 2 * ls
        b = _unit(flag_i, m, 1)
        lenq, lenh = m << 2, m >> 1
        pos = k % m
        first = pos < lenh
        coeff[s0, ~first] = b
        coeff[s1, first] = b
        j = pos[first]
        w = cmul(np.full(j.shape, b), pows[(rg[j] % lenq) * (dim // lenq)])
        coeff[s2, first] = w
        coeff[s1, np.nonzero(first)[0] + lenh] = -w
        m <<= 1
    return coeff


def _collapse_encoding(c1, top, nl, nz, ls, slots):
    """coeff_encoding_collapse's fold of nl layers from layer index top down: after layer l the vectors are
    cs[2u] = c1[top - l] rot(temp[u], -sh) + c1[top - l + 2 ls] rot(temp[u - 1], sh) (two terms, so their order does
    not change the sum) and cs[2u + 1] = c1[top - l + ls] temp[u]"""
    cs = np.zeros((nz, slots), np.complex128)
    cs[0], cs[1], cs[2] = c1[top], c1[top + ls], c1[top + 2 * ls]
    k = np.arange(slots)
    for l in range(1, nl):
        temp = cs
        cs = np.zeros((nz, slots), np.complex128)
        sh = 1 << (top - l)
        nu = (1 << (l + 1)) - 1
        t = temp[:nu]
        A = cmul(c1[top - l][None, :], t[:, (k - sh) % slots])
        Bv = cmul(c1[top - l + ls][None, :], t)
        Cv = cmul(c1[top - l + 2 * ls][None, :], t[:, (k + sh) % slots])
        cs[0:2 * nu:2] += A
        cs[1:2 * nu:2] += Bv
        cs[2:2 * nu + 1:2] += Cv
    return cs


def coeff_encoding_collapse(pows, rg, level_budget, flag_i):
    """OpenFHE CoeffEncodingCollapse -> [s][d][k], s = 0..budget (0: the remainder stage when the layers do not divide
    log2 slots) (bts_setup.rs:437-500)"""
    slots = len(rg)
    if slots == 0 or level_budget == 0:
        raise ValueError("coeff_encoding_collapse: empty rotGroup or zero budget")
    ls = slots.bit_length() - 1
    layers, _rows, rem = select_layers(ls, level_budget)
    flag_rem = 1 if rem else 0
    nr, nr_rem = (1 << (layers + 1)) - 1, (1 << (rem + 1)) - 1
    c1 = coeff_encoding_one_level(pows, rg, flag_i)
    out = [None] * level_budget
    if layers > 0:
        for s in range(level_budget - 1, flag_rem - 1, -1):
            back = (level_budget - 1 - s) * layers + 1
            if ls < back:
                raise ValueError("coeff_encoding_collapse: top can not be negative")
            top = ls - (level_budget - 1 - s) * layers - 1
            out[s] = _collapse_encoding(c1, top, layers, nr, ls, slots)
    if flag_rem:
        top = ls - (level_budget - 1) * layers - 1
        out[0] = _collapse_encoding(c1, top, rem, nr_rem, ls, slots)
    for s in range(level_budget):
        if out[s] is None:
            out[s] = np.zeros((nr, slots), np.complex128)
    return out


def _collapse_decoding(c1, s, layers, nl, nz, ls, slots):
    """coeff_decoding_collapse's fold: each vector receives up to three terms, added in the order t = 0, 1, 2"""
    base = s * layers
    cs = np.zeros((nz, slots), np.complex128)
    cs[0], cs[1], cs[2] = c1[base], c1[ls + base], c1[2 * ls + base]
    for l in range(1, nl):
        temp = cs
        cs = np.zeros((nz, slots), np.complex128)
        nu = (1 << (l + 1)) - 1
        for t, shift in enumerate((0, 1 << l, 1 << (l + 1))):
            cs[shift:shift + nu] += cmul(c1[base + l + t * ls][None, :], temp[:nu])
    return cs


def coeff_decoding_collapse(pows, rg, level_budget, flag_i):
    """OpenFHE CoeffDecodingCollapse -> [s][d][k], s = 0..budget (the last: the remainder stage) (bts_setup.rs:
    502-552)"""
    slots = len(rg)
    if slots == 0 or level_budget == 0:
        raise ValueError("coeff_decoding_collapse: empty rotGroup or zero budget")
    ls = slots.bit_length() - 1
    layers, rows, rem = select_layers(ls, level_budget)
    nr, nr_rem = (1 << (layers + 1)) - 1, (1 << (rem + 1)) - 1
    c1 = coeff_decoding_one_level(pows, rg, flag_i)
    out = [np.zeros((nr, slots), np.complex128) for _ in range(level_budget)]
    if layers > 0:
        for s in range(rows):
            out[s] = _collapse_decoding(c1, s, layers, layers, nr, ls, slots)
    if rem:
        out[rows] = _collapse_decoding(c1, rows, layers, rem, nr_rem, ls, slots)
    return out


def rotate_left(a, r):
    """OpenFHE Rotate(a, r): out[k] = a[(k + r) mod len]"""
    n = len(a)
    return np.roll(a, -(r % n)) if n else a


class FftStage:
    """One collapsed-FFT stage (OpenFHE stage index s): y[k] = sum_d diags[d][k] x[(k + (d - center) stride) mod len],
    center = (num_diags - 1) / 2; b giant (outer) and g baby (inner) steps (bts_setup.rs:556-613)."""

    def __init__(self, s, stride, b, g, diags):
        self.s, self.stride, self.b, self.g, self.diags = s, stride, b, g, diags

    def num_diags(self):
        return len(self.diags)

    def center(self):
        return (len(self.diags) - 1) // 2

    def bsgs_diag(self, idx):
        """the plaintext OpenFHE encodes for diagonal idx = g i + j: Rotate(diag, -g i stride)"""
        i = idx // self.g
        return rotate_left(self.diags[idx], -self.g * i * self.stride)

    def rot_in(self, red):
        h = (len(self.diags) + 1) // 2
        return [reduce_rotation((j - h + 1) * self.stride, red) for j in range(self.g)]

    def rot_out(self, m4):
        return [reduce_rotation(self.g * i * self.stride, m4) for i in range(self.b)]

    def apply(self, x):
        c = self.center()
        y = np.zeros(len(x), np.complex128)
        for d, dv in enumerate(self.diags):
            y += cmul(dv, rotate_left(x, (d - c) * self.stride))
        return y


class FidesStage:
    """One stage in FIDESlib's layout (bts_setup.rs:822-836): pts[i b_step + j] multiplies rot(x, rot_in[j]) inside
    giant step i, which is then rotated by rot_out[i]; b_step = OpenFHE g, g_step = OpenFHE b; every plaintext is the
    OpenFHE BSGS plaintext rotated left by pt_rotation."""

    def __init__(self, num_diags, b_step, g_step, rot_in, rot_out, pt_rotation, pts):
        self.num_diags, self.b_step, self.g_step = num_diags, b_step, g_step
        self.rot_in, self.rot_out, self.pt_rotation, self.pts = rot_in, rot_out, pt_rotation, pts


class BtsFactors:
    """All CtS and StC factors of one slot count (bts_setup.rs:629-640): cts[s] / stc[s] by OpenFHE stage index (CtS
    runs s = budget - 1 down to 0, StC s = 0 up)."""

    def __init__(self, n, slots, enc, dec, cts, stc):
        self.n, self.slots, self.enc, self.dec, self.cts, self.stc = n, slots, enc, dec, cts, stc

    def m4(self):
        return self.n // 2

    def cts_rotation_indices(self):
        """OpenFHE FindCoeffsToSlotsRotationIndices, duplicates kept, in its order (bts_setup.rs:722-752)"""
        p, v = self.enc, []
        flag_rem = 1 if p.rem_collapse else 0
        for s in range(p.level_budget - 1, flag_rem - 1, -1):
            sf = 1 << ((s - flag_rem) * p.layers_collapse + p.rem_collapse)
            half = 1 - (p.num_rotations + 1) // 2
            v += [reduce_rotation(j * sf, self.slots) for j in range(half, p.g + half)]
            v += [reduce_rotation(p.g * i * sf, self.m4()) for i in range(p.b)]
        if flag_rem:
            half = 1 - (p.num_rotations_rem + 1) // 2
            v += [reduce_rotation(j, self.slots) for j in range(half, p.g_rem + half)]
            v += [reduce_rotation(p.g_rem * i, self.m4()) for i in range(p.b_rem)]
        self._push_sparse(v)
        return v

    def stc_rotation_indices(self):
        """OpenFHE FindSlotsToCoeffsRotationIndices (bts_setup.rs:754-782)"""
        p, v = self.dec, []
        flag_rem = 1 if p.rem_collapse else 0
        for s in range(p.level_budget - flag_rem):
            sf = 1 << (s * p.layers_collapse)
            half = 1 - (p.num_rotations + 1) // 2
            v += [reduce_rotation(j * sf, self.m4()) for j in range(half, p.g + half)]
            v += [reduce_rotation(p.g * i * sf, self.m4()) for i in range(p.b)]
        if flag_rem:
            sf = 1 << ((p.level_budget - 1) * p.layers_collapse)
            half = 1 - (p.num_rotations_rem + 1) // 2
            v += [reduce_rotation(j * sf, self.m4()) for j in range(half, p.g_rem + half)]
            v += [reduce_rotation(p.g_rem * i * sf, self.m4()) for i in range(p.b_rem)]
        self._push_sparse(v)
        return v

    def _push_sparse(self, v):
        m, mm = 4 * self.slots, 2 * self.n
        if m != mm:
            j = 1
            while j < mm // m:
                v.append(j * self.slots)
                j <<= 1

    def bootstrap_rotation_indices(self):
        """OpenFHE FindBootstrapRotationIndices: the sorted CtS and StC rotations without 0 and M / 4"""
        s = set(self.cts_rotation_indices()) | set(self.stc_rotation_indices())
        s.discard(0)
        s.discard(self.m4())
        return sorted(s)

    def fides_layout(self):
        """FIDESlib GetBootstrapIndexes + ltFriendly (bts_setup.rs:852-940): rot_in from 0 at its first-step
        spacing, rot_out re-based on giant step 0, every plaintext pre-rotated by the running sum of those offsets;
        the last StC stage's rot_out pays the accumulated offset. Returns (cts stages in evaluation order, stc stages,
        the accumulated offset)."""
        m4 = self.m4()
        modv = min(2 * self.slots, self.n // 2)
        cmod = lambda a, m: int(math.fmod(a, m))  # C's % (the dividend's sign)

        def build(st, red_in):
            ri = list(st.rot_in(red_in))
            ro = list(st.rot_out(m4))
            off = ri[0]
            return [x - off for x in ri], [x + off for x in ro]

        def fix_in(ri, b_step, g_step, nd):
            for i in range(g_step):
                for j in range(1, b_step):
                    if i * b_step + j < nd and len(ri) > 1 and ri[j] - ri[j - 1] != ri[1] - ri[0]:
                        ri[j] = ri[j - 1] + ri[1] - ri[0]

        acc_load = 0
        out = []
        stages = [(st, self.slots) for st in reversed(self.cts)] + [(st, m4) for st in self.stc]
        for si, (st, red_in) in enumerate(stages):
            ri, ro = build(st, red_in)
            off = ro[0]
            ro = [ro[0]] + [cmod(x - off, modv) for x in ro[1:]]
            fix_in(ri, st.g, st.b, st.num_diags())
            acc_load += ro[0]
            ro[0] = 0
            rot = reduce_rotation(-acc_load, m4)
            pts = [rotate_left(st.bsgs_diag(d), rot) for d in range(st.num_diags())]
            if si == len(stages) - 1:
                ro = [cmod(acc_load, modv)] + [cmod(x + acc_load, modv) for x in ro[1:]]
            out.append(FidesStage(st.num_diags(), st.g, st.b, ri, ro, rot, pts))
        return out[:len(self.cts)], out[len(self.cts):], acc_load


def cts_stc_factors(n, slots, level_budget, dim1, scale_enc, scale_dec):
    """The collapsed-FFT factors of EvalBootstrapSetup(levelBudget, dim1, slots) for ring dimension n (bts_setup.rs:
    642-720): scale_enc folded into CtS stage 0, scale_dec into the last StC stage; budgets clamped to
    [1, log2 slots]; the single-LT route (budget {1, 1}) is refused."""
    if n & (n - 1) or n < 8:
        raise ValueError(f"cts_stc_factors: ring dimension n={n}")
    m_big = 2 * n
    slots = slots or m_big // 4
    if slots & (slots - 1) or slots > m_big // 4 or slots < 2:
        raise ValueError(f"cts_stc_factors: slots={slots} for n={n}")
    log_slots = 1 if slots < 3 else slots.bit_length() - 1
    budget = [min(max(b, 1), log_slots) for b in level_budget]
    if budget == [1, 1]:
        raise ValueError("cts_stc_factors: level budget {1,1} is the single-LT route")
    enc = CollapsedFftParams(slots, budget[0], dim1[0])
    dec = CollapsedFftParams(slots, budget[1], dim1[1])
    m = 4 * slots
    rg = rot_group(slots, m)
    pows = ksi_pows(m)
    full = slots == m_big // 4

    flag_rem = 1 if enc.rem_collapse else 0
    ce = coeff_encoding_collapse(pows, rg, enc.level_budget, False)
    cei = None if full else coeff_encoding_collapse(pows, rg, enc.level_budget, True)
    cts = []
    for s in range(enc.level_budget):
        rem_stage = flag_rem and s == 0
        b, g, nr = (enc.b_rem, enc.g_rem, enc.num_rotations_rem) if rem_stage else (enc.b, enc.g, enc.num_rotations)
        stride = 1 if rem_stage else 1 << ((s - flag_rem) * enc.layers_collapse + enc.rem_collapse)
        diags = []
        for d in range(nr):
            v = ce[s][d].copy()
            if cei is not None:
                v = np.concatenate([v, cei[s][d]])
            if s == 0:
                v = cscale(v, scale_enc)
            diags.append(v)
        cts.append(FftStage(s, stride, b, g, diags))

    flag_rem = 1 if dec.rem_collapse else 0
    cd = coeff_decoding_collapse(pows, rg, dec.level_budget, False)
    cdi = None if full else coeff_decoding_collapse(pows, rg, dec.level_budget, True)
    stc = []
    for s in range(dec.level_budget):
        rem_stage = flag_rem and s == dec.level_budget - 1
        b, g, nr = (dec.b_rem, dec.g_rem, dec.num_rotations_rem) if rem_stage else (dec.b, dec.g, dec.num_rotations)
        stride = 1 << (s * dec.layers_collapse)
        diags = []
        for d in range(nr):
            v = cd[s][d].copy()
            if cdi is not None:
                v = np.concatenate([v, cdi[s][d]])
            if s == dec.level_budget - 1:
                v = cscale(v, scale_dec)
            diags.append(v)
        stc.append(FftStage(s, stride, b, g, diags))
    return BtsFactors(n, slots, enc, dec, cts, stc)
