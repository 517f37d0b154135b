"""perseus_amd/bts_setup.py, the restatement of the reference's bootstrap constants, pinned on the CPU:
- the reference's own known answers: the stage metadata of the N = 2^16 full-slot factors at budgets [4, 3]
  (crates/pc-core/tests/oracle_bts.rs:57-64), its rotation set (:91-100), OpenFHE's ReduceRotation quirk;
- what the mathematics fixes: the StC stages compose to U0 brev and the CtS stages to brev(U0^H) (unnormalised) at
  every collapse shape (oracle_bts.rs:145-197, U0[i][j] = zeta^(j 5^i) summed directly); the BSGS form (pre-rotated
  diagonals, rot_in / rot_out) and FIDESlib's layout compute the stages' maps (:207-269);
- an independent construction (tests/special_fft.py: the special FFT's butterfly layers grouped into levels): each
  CtS stage is 2^layers times the matching level, each StC stage equal to it;
- the EvalMod table: the Chebyshev interpolant against numpy's (c0 halved), and after its three double angles against
  sin(2 pi 32 y) / (2 pi); the double-angle constants against the closed form (2 pi)^(-2^(j - 3)).
A plausible slip (a transposed twiddle index, a dropped conjugation, a wrong shift sign, a swapped baby / giant
count) moves one of the maps by O(1) and fails these checks."""
import math

import numpy as np
import pytest

from perseus_amd import bootstrap as B
from perseus_amd import bts_setup as S
from tests import special_fft as SF


def maxd(a, b):
    return float(np.abs(np.asarray(a) - np.asarray(b)).max())


def test_stage_metadata_of_the_c5_shape():
    f = S.cts_stc_factors(1 << 16, 1 << 15, [4, 3], [0, 0], 1.0, 1.0)
    e, d = f.enc, f.dec
    assert (e.layers_collapse, e.rem_collapse, e.num_rotations, e.b, e.g, e.num_rotations_rem, e.b_rem, e.g_rem) == \
        (4, 3, 31, 2, 16, 15, 2, 8)
    assert (d.layers_collapse, d.rem_collapse, d.num_rotations, d.b, d.g) == (5, 0, 63, 4, 16)
    assert [st.stride for st in f.cts] == [1, 8, 128, 2048] and [st.stride for st in f.stc] == [1, 32, 1024]
    rots = f.bootstrap_rotation_indices()
    assert all(0 < r < 1 << 15 for r in rots)
    for k in range(1, 16):
        assert k * 2048 in rots
    cts, stc, acc = f.fides_layout()
    assert [st.rot_in[:3] for st in cts] == [[0, 2048, 4096], [0, 128, 256], [0, 8, 16], [0, 1, 2]]
    assert all(st.rot_out[0] == 0 for st in cts + stc[:-1])
    assert stc[-1].rot_out[0] == acc % (1 << 15)


def test_reduce_rotation_and_select_layers():
    assert S.reduce_rotation(-(1 << 15), 1 << 15) == 1 << 15  # OpenFHE keeps slots for a negative multiple
    assert S.reduce_rotation(-5, 16) == 11 and S.reduce_rotation(37, 16) == 5 and S.reduce_rotation(-5, 12) == 7
    assert S.select_layers(15, 4) == (4, 3, 3) and S.select_layers(15, 3) == (5, 3, 0)
    assert S.select_layers(15, 1) == (15, 1, 0) and S.select_layers(7, 7) == (1, 7, 0)
    assert S.select_layers(4, 3) == (1, 2, 2)
    for ls in range(1, 16):
        for b in range(1, ls + 1):
            layers, rows, rem = S.select_layers(ls, b)
            assert rows * layers + rem == ls and rem >= 0  # the remainder may exceed layers (select_layers(4, 3))


def u0(x, slots):
    """OpenFHE's U0 x, U0[i][j] = ksi^(j 5^i), summed directly"""
    m = 4 * slots
    rg = S.rot_group(slots, m)
    j = np.arange(slots)
    return np.array([np.sum(np.exp(2j * np.pi * ((j * rg[i]) % m) / m) * x) for i in range(slots)])


def u0h(x, slots):
    m = 4 * slots
    rg = S.rot_group(slots, m)
    out = np.zeros(slots, complex)
    for i in range(slots):
        out += np.exp(-2j * np.pi * ((np.arange(slots) * rg[i]) % m) / m) * x[i]
    return out


@pytest.mark.parametrize("budget", [[2, 2], [3, 3], [4, 2], [7, 7], [1, 3], [3, 1], [4, 3]])
def test_stages_compose_to_the_dft(budget):
    n = 1 << 8
    slots = n // 2
    br = SF.bitrev(slots)
    rng = np.random.default_rng(5)
    x = rng.uniform(-0.5, 0.5, slots) + 1j * rng.uniform(-0.5, 0.5, slots)
    f = S.cts_stc_factors(n, slots, budget, [0, 0], 1.0, 1.0)
    y = x
    for st in f.stc:
        y = st.apply(y)
    assert maxd(y, u0(x[br], slots)) < 1e-9
    z = x
    for st in reversed(f.cts):
        z = st.apply(z)
    assert maxd(z, u0h(x, slots)[br]) < 1e-9


@pytest.mark.parametrize("budget", [[4, 3], [3, 3], [2, 4]])
def test_bsgs_and_fides_layout(budget):
    n = 1 << 9
    slots = n // 2
    rng = np.random.default_rng(11)
    x = rng.uniform(-0.5, 0.5, slots) + 1j * rng.uniform(-0.5, 0.5, slots)
    f = S.cts_stc_factors(n, slots, budget, [0, 0], 0.5, 2.0)
    chain = x
    for st in list(reversed(f.cts)) + f.stc:
        rin, rout = st.rot_in(slots), st.rot_out(slots)
        y = np.zeros(slots, complex)
        for i in range(st.b):
            inner = np.zeros(slots, complex)
            for j in range(st.g):
                idx = st.g * i + j
                if idx < st.num_diags():
                    inner += st.bsgs_diag(idx) * S.rotate_left(chain, rin[j])
            y += S.rotate_left(inner, rout[i])
        want = st.apply(chain)
        assert maxd(y, want) < 1e-9, f"stage s={st.s}: BSGS != the stage"
        chain = want
    cts, stc, _ = f.fides_layout()
    fx = x
    for st in cts + stc:
        fx = B.LtPlan(st, slots).apply(fx)
    assert maxd(fx, chain) < 1e-9, "FIDESlib's layout != OpenFHE's chain"


def test_stages_against_the_independent_levels():
    """the reference's stage s as a map = 2^layers x this repository's own CtS level (inverse layers with their
    halves), = its StC level; the same grouping of layers ([4, 4, 4, 3] and [5, 5, 5] at 2^15 slots; here 2^8 slots,
    [2, 2, 2, 2] and [3, 3, 2])"""
    n = 1 << 9
    slots = n // 2
    f = S.cts_stc_factors(n, slots, [4, 3], [0, 0], 1.0, 1.0)
    sizes_c = []
    for st in reversed(f.cts):  # evaluation order: the stage's layer count from its number of diagonals
        sizes_c.append((len(st.diags) + 1).bit_length() - 2)
    sizes_s = [(len(st.diags) + 1).bit_length() - 2 for st in f.stc]
    assert sizes_c == [2, 2, 2, 2] and sizes_s == [3, 3, 2]
    rng = np.random.default_rng(2)
    x = rng.normal(size=slots) + 1j * rng.normal(size=slots)
    for st, lv, L in zip(reversed(f.cts), SF.cts_levels(slots, sizes_c), sizes_c):
        assert maxd(st.apply(x), (1 << L) * SF.apply_diags(lv, x)) < 1e-9
    for st, lv in zip(f.stc, SF.stc_levels(slots, sizes_s)):
        assert maxd(st.apply(x), SF.apply_diags(lv, x)) < 1e-9
    # the independent levels themselves against the canonical embedding summed directly
    w = rng.normal(size=slots) + 1j * rng.normal(size=slots)
    y = w[SF.bitrev(slots)]
    for lv in SF.stc_levels(slots, sizes_s):
        y = SF.apply_diags(lv, y)
    assert maxd(y, u0(w, slots)) < 1e-9


def test_evalmod_table():
    t = S.evalmod_k32_low()
    assert len(t) == 60
    f = lambda y: (2 * np.pi) ** (-1 / 8) * np.cos(2 * np.pi * (32 * y - 0.25) / 8)
    ref = np.polynomial.chebyshev.chebinterpolate(f, 59)
    assert abs(t[0] / 2 - ref[0]) < 1e-15 and maxd(t[1:], ref[1:]) < 1e-14
    em = B.EvalModPlan()
    u = np.linspace(-1, 1, 20001)
    assert maxd(em.plain(u), np.sin(2 * np.pi * 32 * u) / (2 * np.pi)) < 1e-11
    for j in (1, 2, 3):
        assert math.isclose(S.double_angle_scalar(j, 3), -(2 * math.pi) ** (-2.0 ** (j - 3)), rel_tol=1e-15)
    # the prefactor: the series alone is (2 pi)^(-1/8) cos(...) on [-1, 1]
    assert maxd(B.cheb_eval(em.c, u), f(u)) < 1e-12
    for g in (8, 16, 32):
        c = em.c[: 2 * g]
        q, r = B.cheb_split(c, g)
        Tg = np.polynomial.chebyshev.chebval(u, np.eye(g + 1)[g])
        assert maxd(B.cheb_eval(q, u) * Tg + B.cheb_eval(r, u), B.cheb_eval(c, u)) < 1e-12


def test_cheb_interp_parity_and_constants():
    c = S.cheb_interp(9, 1, lambda y: y ** 3)  # odd: x^3 = (3 T1 + T3) / 4
    assert maxd(c, [0, 0.75, 0, 0.25, 0, 0, 0, 0, 0, 0]) < 1e-14
    c = S.cheb_interp(6, 0, lambda y: y * y)  # even: x^2 = (T0 + T2) / 2, c0 not halved: 1
    assert maxd(c, [1.0, 0, 0.5, 0, 0, 0, 0]) < 1e-14
