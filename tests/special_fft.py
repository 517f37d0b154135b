"""An independent construction of the bootstrap's linear transforms, test infrastructure only: the decoding map of
CKKS (z_j = sum_i w_i zeta^(5^j i)) factored into log2(N/2) butterfly layers written directly from the special FFT,
grouped into levels as diagonals {offset: vector}, and a generic baby-step giant-step split of such a level. The tests
use it to pin perseus_amd/bts_setup.py's restatement of the reference's collapsed-FFT factors: each reference stage,
as a linear map, is 2^layers times the matching level here (CoeffToSlot) or equal to it (SlotToCoeff)."""
import math

import numpy as np


def rot_group(n):
    """5^j mod 4n, j < n: slot j sits at the root zeta^(5^j), zeta = exp(2 pi i / 4n)."""
    g = np.empty(n, np.int64)
    v = 1
    for j in range(n):
        g[j] = v
        v = v * 5 % (4 * n)
    return g


def _layer_w(n, ln):
    """The twiddles of the butterfly layer of blocks of 2^ln slots, per slot of the first half of each block."""
    m, length = 4 * n, 1 << ln
    lenh, lenq = length >> 1, length << 2
    k = np.arange(n)
    pos = k % length
    first = pos < lenh
    j = np.where(first, pos, pos - lenh)
    idx = (rot_group(n)[j] % lenq) * (m // lenq)
    return first, np.exp(2j * np.pi * idx / m), lenh


def layer(n, ln):
    """Decoding layer (blocks of 2^ln): u, v -> u + w v, u - w v, as diagonals {offset: vector} over n slots
    (y[k] = sum_d D_d[k] x[(k + d) mod n])."""
    first, w, lenh = _layer_w(n, ln)
    return {0: np.where(first, 1.0, -w).astype(complex), lenh: np.where(first, w, 0).astype(complex),
            -lenh: np.where(first, 0, 1).astype(complex)}


def layer_inv(n, ln):
    """Inverse of `layer`: y_top, y_bot -> (y_top + y_bot) / 2, (y_top - y_bot) / (2 w)."""
    first, w, lenh = _layer_w(n, ln)
    iw = 1.0 / (2.0 * w)
    return {0: np.where(first, 0.5, -iw).astype(complex), lenh: np.where(first, 0.5, 0).astype(complex),
            -lenh: np.where(first, 0, iw).astype(complex)}


def _norm(d, n):
    d %= n
    return d - n if d > n // 2 else d


def compose(a, b, n):
    """Diagonals of A o B (B applied first)."""
    out = {}
    for da, va in a.items():
        for db, vb in b.items():
            d = _norm(da + db, n)
            t = va * np.roll(vb, -da)
            out[d] = out[d] + t if d in out else t
    return out


def apply_diags(diags, x):
    """y = sum_d D_d * rot(x, d) on plain slot vectors (rot(x, d)[k] = x[k + d])."""
    y = np.zeros_like(x, dtype=complex)
    for d, v in diags.items():
        y += v * np.roll(x, -d)
    return y


def bitrev(n):
    b = n.bit_length() - 1
    return np.array([int(format(i, f"0{b}b")[::-1], 2) for i in range(n)], np.int64)


def cts_levels(n, sizes):
    """The CoeffToSlot levels: the inverse layers applied from blocks of n down to blocks of 2, grouped `sizes` (sum =
    log2 n) in order of application; their product is the inverse decoding map up to the bit reversal."""
    assert sum(sizes) == n.bit_length() - 1
    lns = list(range(n.bit_length() - 1, 0, -1))
    out, i = [], 0
    for s in sizes:
        acc = None
        for ln in lns[i:i + s]:
            L = layer_inv(n, ln)
            acc = L if acc is None else compose(L, acc, n)
        out.append(acc)
        i += s
    return out


def stc_levels(n, sizes):
    """The SlotToCoeff levels: the decoding layers from blocks of 2 up to blocks of n, grouped `sizes`."""
    assert sum(sizes) == n.bit_length() - 1
    lns = list(range(1, n.bit_length()))
    out, i = [], 0
    for s in sizes:
        acc = None
        for ln in lns[i:i + s]:
            L = layer(n, ln)
            acc = L if acc is None else compose(L, acc, n)
        out.append(acc)
        i += s
    return out


class BsgsPlan:
    """A level y = sum_d D_d rot(x, d), offsets d = k s with k in [k0, k1], as baby-step giant-step: k - k0 = B j + i,
    y = sum_j rot(sum_i D'_{j,i} rot(x, i s), g_j s), g_j = B j + k0, D'_{j,i} = rot(D_{(g_j + i) s}, -g_j s)."""

    def __init__(self, diags, n, B=None):
        offs = [d for d, v in diags.items() if np.abs(v).max() > 0]
        s = 0
        for d in offs:
            s = math.gcd(s, abs(d))
        s = s or 1
        ks = sorted(d // s for d in offs)
        k0, k1 = ks[0], ks[-1]
        width = k1 - k0 + 1
        self.n, self.s = n, s
        self.B = B or (1 << max(1, (width.bit_length() + 1) // 2))
        self.G = -(-width // self.B)
        self.baby = [i * s for i in range(self.B)]
        self.giant = [(self.B * j + k0) * s for j in range(self.G)]
        self.pts = []
        for j in range(self.G):
            row = []
            for i in range(self.B):
                k = self.B * j + k0 + i
                v = diags.get(k * s) if k <= k1 else None
                row.append(None if v is None or np.abs(v).max() == 0 else np.roll(v, self.giant[j]))
            self.pts.append(row)

    def apply(self, x):
        rots = [np.roll(x, -b) for b in self.baby]
        y = np.zeros(self.n, complex)
        for j in range(self.G):
            acc = np.zeros(self.n, complex)
            for i in range(self.B):
                if self.pts[j][i] is not None:
                    acc += self.pts[j][i] * rots[i]
            y += np.roll(acc, -self.giant[j])
        return y
