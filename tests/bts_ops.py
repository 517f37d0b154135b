"""The bootstrap composite's operations on the oracle (test infrastructure): the same interface as
perseus_amd.bootstrap.GpuOps over numpy ciphertexts [2][rows][N], each operation the oracle's pinned counterpart
(tests/twin.py key switches and rescale, oracle/em.py element-wise kernels and pt_dot, oracle/bts.py mod_raise), so
that the composite run on both gives the same words.
"""
import numpy as np

from oracle import bts as ob
from oracle import em
from perseus_amd import bts
from perseus_amd.bootstrap import compact_rows


class OracleOps:
    def __init__(self, oc, primes, seeds, bs, levels, conj, relin_seed, relin_b):
        self.oc = oc
        self.q = [int(p) for p in primes]
        self.R, self.N = oc.rows, oc.n
        self.seeds, self.bs, self.levels, self.conj_key = seeds, bs, levels, conj
        self.relin_seed, self.relin_b = relin_seed, relin_b
        self.gal = None
        self.level_i = 0
        self.kmax = 2  # the leaves' batched rescales taken two at a time, one after the other
        self.mr = bts.mod_raise_consts(self.q, 1)

    def set_galois(self, gal):
        self.gal = gal

    def begin(self):
        self.level_i = 0

    # handles: (array [count][2][R][N], index)
    def alloc(self, count=1):
        return (np.zeros((count, 2, self.R, self.N), np.uint32), 0)

    def item(self, h, i):
        return (h[0], h[1] + i)

    @staticmethod
    def get(h):
        return h[0][h[1]]

    def _qq(self, top):
        return np.array(self.q[: top + 1], np.uint64)[None, :, None]

    def copy(self, dst, src, top):
        self.get(dst)[:, : top + 1] = self.get(src)[:, : top + 1]

    def add(self, out, a, b, top, sub):
        q = self._qq(top)
        x, y = self.get(a)[:, : top + 1].astype(np.uint64), self.get(b)[:, : top + 1].astype(np.uint64)
        self.get(out)[:, : top + 1] = ((x + q - y) % q if sub else (x + y) % q).astype(np.uint32)

    def mul_const(self, out, x, top, k):
        kr = np.array([int(k) % p for p in self.q[: top + 1]], np.uint64)[None, :, None]
        self.get(out)[:, : top + 1] = (self.get(x)[:, : top + 1].astype(np.uint64) * kr % self._qq(top)).astype(
            np.uint32)

    def add_const(self, x, top, k):
        kr = np.array([int(k) % p for p in self.q], np.uint32)
        self.get(x)[:, : top + 1] = em.add_const(self.q[: top + 1], self.get(x)[None, :, : top + 1], kr[: top + 1])[0]

    def wsum(self, out, srcs, top, ks, k0):
        w = np.array([[k % p for p in self.q[: top + 1]] for k in ks], np.uint64)
        kr = np.array([k0 % p for p in self.q[: top + 1]], np.uint64)
        self.get(out)[:, : top + 1] = em.wsum(self.q[: top + 1], [self.get(x)[None, :, : top + 1] for x in srcs], w,
                                              kr)[0]

    def mul_pt(self, out, x, top, pt):
        self.get(out)[:, : top + 1] = (self.get(x)[:, : top + 1].astype(np.uint64) *
                                       pt[None, : top + 1].astype(np.uint64) % self._qq(top)).astype(np.uint32)

    def plaintext(self, coef_rows, top, s=0):
        ids = list(range(top + 1))
        return compact_rows(self.oc.ntt_fwd(np.ascontiguousarray(coef_rows[: top + 1], np.uint32).copy(), ids), s)

    def plaintext_ext(self, coef_rows, top, s=0):  # full rows: the compact form is the GPU's storage of the same values
        kp = self.R - len(self.q)
        ids = list(range(top + 1)) + [len(self.q) + j for j in range(kp)]
        return self.oc.ntt_fwd(np.ascontiguousarray(coef_rows[: top + 1 + kp], np.uint32).copy(), ids)

    def cts(self, res, x, top, pts, B, G, s=0):
        kp = self.R - len(self.q)
        zero = np.zeros((top + 1 + kp, self.N), np.uint32)
        full = [zero if p is None else p for p in pts]
        babies = self.levels[self.level_i][0]
        xx = self.get(x)
        digits = self.oc.modup(xx[1], top)
        out = self.oc.cts_fused(xx[None], digits[None], top, B, G, full, [self.gal[r] for r in babies],
                                seeds=self.seeds[babies] if babies else None, bs=[self.bs[r] for r in babies])[0]
        res[0][res[1]: res[1] + G] = out

    def moddown(self, out, ext, top):
        self.get(out)[:] = self.oc.moddown(self.get(ext).copy(), top)

    def pt_dot(self, res, rots, top, pts, B, G, s=0):
        zero = np.zeros((top + 1, self.N >> s), np.uint32)
        full = [zero if p is None else p for p in pts]
        rot = rots[0][rots[1]: rots[1] + B][None, :, :, : top + 1]
        enc = (0x7F000000 | s) if s else 0xFFFFFFFF
        out = em.pt_dot(self.q[: top + 1], rot, full, B, G, B * G, enc, list(range(top + 1)))
        res[0][res[1]: res[1] + G, :, : top + 1] = out[0]

    def rotate(self, out, x, top, step):
        r = self.conj_key if step == "conj" else self.levels[self.level_i][1][step]
        self.get(out)[:] = self.oc.rotate(self.get(x), top, self.seeds[r], self.bs[r], self.gal[r])

    def rotate_many(self, out, xs, top, steps, onto):
        r = [self.levels[self.level_i][1][g] for g in steps]
        self.get(out)[:] = self.oc.rotate_many([self.get(x) for x in xs], top, self.seeds[r], [self.bs[i] for i in r],
                                               [self.gal[i] for i in r], onto=None if onto is None else self.get(onto))

    def rotate_many_rescale(self, out, xs, top, steps, onto):
        r = [self.levels[self.level_i][1][g] for g in steps]
        self.get(out)[:] = self.oc.rotate_many([self.get(x) for x in xs], top, self.seeds[r], [self.bs[i] for i in r],
                                               [self.gal[i] for i in r], onto=None if onto is None else self.get(onto),
                                               rescale=True)

    def hoisted(self, outs, x, top, steps):
        babies = self.levels[self.level_i][0]
        res = self.oc.rotate_hoisted(self.get(x), top, self.seeds[babies], [self.bs[r] for r in babies],
                                     [self.gal[r] for r in babies])
        for i, r in enumerate(res):
            self.get(self.item(outs, i))[:] = r

    def level_done(self):
        self.level_i += 1

    def fork(self, other):
        pass

    def join(self, other):
        pass

    def mul_relin(self, out, a, b, top):
        self.get(out)[:] = self.oc.mul_relin(self.get(a), self.get(b), top, self.relin_seed, self.relin_b)

    def mul_relin_rescale(self, out, a, b, top, twice=False):
        x = self.get(a)
        if twice:  # the doubling as the composite's add(a, a) would make it, then the product
            x = x.copy()
            self.add((x[None], 0), (x[None], 0), (x[None], 0), top, False)
        self.get(out)[:] = self.oc.mul_relin_rescale(x, self.get(b), top, self.relin_seed, self.relin_b)

    def mul_list(self, out, a, b, top, twice=False):
        for j in range(len(a)):
            self.mul_relin_rescale(self.item(out, j), a[j], b[j], top, twice)

    sum_pairs = 8

    def mul_sum_list(self, out, groups, top, adds=None, sub=0, kmuls=None, twice=False):
        for j, g in enumerate(groups):
            y = None if adds is None or adds[j] is None else self.get(adds[j])
            k = None if kmuls is None else kmuls[j]
            self.get(self.item(out, j))[:] = self.oc.mul_sum_relin_rescale(
                [(self.get(a), self.get(b)) for a, b in g], top, self.relin_seed, self.relin_b, y, (sub >> j) & 1, k,
                twice)

    def rescale2(self, out, x, top, count=1):
        for i in range(count):
            self.get(self.item(out, i))[:] = self.oc.rescale(self.get(self.item(x, i)).copy(), top, 2)

    def mod_raise(self, out, x, top):
        o = self.get(out)
        o[:] = 0
        qhatinv, qhat = self.mr
        for part in range(2):
            row0 = self.oc.ntt_inv(self.get(x)[part, :1].copy(), [0])
            rows = np.zeros((top + 1, self.N), np.uint32)
            rows[0] = row0[0]
            rows[1:] = ob.mod_raise(self.q, rows, 1, 1, top + 1, qhatinv, qhat)
            o[part, : top + 1] = self.oc.ntt_fwd(rows, list(range(top + 1)))
