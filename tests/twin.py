"""ctypes bindings of the CPU twin (oracle/libtwin.so): the oracle of every parity test.

Test infrastructure only: the product package (perseus_amd) never imports this module.
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "oracle", "libtwin.so")

u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")


def _load():
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() (or make -C oracle)")
    lib = C.CDLL(LIB_PATH)
    sig = {
        "or_is_prime": (C.c_int, [C.c_uint64]),
        "or_first_prime": (C.c_uint64, [C.c_uint32, C.c_uint64]),
        "or_last_prime": (C.c_uint64, [C.c_uint32, C.c_uint64]),
        "or_previous_prime": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "or_root_of_unity": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "or_invmod": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "or_powmod": (C.c_uint64, [C.c_uint64, C.c_uint64, C.c_uint64]),
        "or_descending_primes": (C.c_int, [C.c_uint32, C.c_uint64, C.c_int, u64p]),
        "or_prime_const": (None, [C.c_uint64, C.c_uint32, C.c_void_p]),
        "or_chacha_block": (None, [u32p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, u32p]),
        "or_kska_expand_row": (None, [u32p, C.c_uint32, C.c_uint32, C.c_uint32, u32p]),
        "or_kska_expand": (C.c_uint32, [u32p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]),
        "or_expand_row": (None, [u32p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, u32p]),
        "or_cts_expand_row": (None, [u32p, C.c_uint32, C.c_uint32, u32p]),
        "or_spru_fft_pass": (None, [f64p, f64p, f64p, C.c_uint32, C.c_uint32, C.c_uint32]),
        "or_spru_scatter": (None, [f64p, f64p, u64p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_double, C.c_uint64,
                                   u32p]),
        "or_kskb_expand_row": (None, [u32p, C.c_uint32, C.c_uint64, C.c_uint32, u64p]),
        "or_prng_new": (C.c_void_p, [u32p, C.c_uint32]),
        "or_prng_free": (None, [C.c_void_p]),
        "or_prng_next_u32": (C.c_uint32, [C.c_void_p]),
        "or_prng_next_u64": (C.c_uint64, [C.c_void_p]),
        "or_prng_uniform_below": (C.c_uint64, [C.c_void_p, C.c_uint64]),
        "or_prng_uniform_f64": (C.c_double, [C.c_void_p]),
        "or_prng_ksk_seed": (None, [C.c_void_p, u32p]),
        "or_sample_sparse_ternary": (C.c_int, [C.c_void_p, C.c_uint32, C.c_uint32, i8p]),
        "or_sample_gaussian": (None, [C.c_void_p, C.c_double, C.c_uint32, i64p]),
        "or_below_accept": (C.c_int, [C.c_uint64, C.c_uint64, C.POINTER(C.c_uint64)]),
        "or_gauss_cdf": (C.c_int, [C.c_double, f64p, C.c_int]),
        "or_gauss_index": (C.c_int, [C.c_double, C.c_double]),
        "or_automorph_slot": (C.c_uint32, [C.c_uint32, C.c_uint32, C.c_uint32]),
        "or_rotation_galois": (C.c_uint64, [C.c_int64, C.c_uint32]),
        "or_galois_inverse": (C.c_uint64, [C.c_uint64, C.c_uint32]),
        "or_ctx_new": (C.c_void_p, [C.c_uint32, u64p, C.c_int, C.c_int, C.c_int]),
        "or_ctx_free": (None, [C.c_void_p]),
        "or_set_threads": (None, [C.c_int]),
        "or_set_cpus": (None, [i32p, C.c_int]),
        "or_set_kska_cache": (None, [C.c_size_t]),
        "or_get_threads": (C.c_int, []),
        "or_ctx_twiddles": (None, [C.c_void_p, C.c_int, u32p, u32p, u32p, u32p]),
        "or_ctx_root": (C.c_uint64, [C.c_void_p, C.c_int]),
        "or_ntt_fwd_rows": (None, [C.c_void_p, u32p, i32p, C.c_int]),
        "or_ntt_inv_rows": (None, [C.c_void_p, u32p, i32p, C.c_int]),
        "or_bconv": (None, [C.c_void_p, C.c_void_p, i32p, C.c_int, C.c_void_p, i32p, C.c_int, C.c_int]),
        "or_live_digits": (C.c_int, [C.c_void_p, C.c_int]),
        "or_digit_of": (C.c_int, [C.c_void_p, C.c_int]),
        "or_modup": (None, [C.c_void_p, u32p, C.c_int, u32p]),
        "or_ks_dot": (None, [C.c_void_p, u32p, u32p, C.c_int, u32p, u32p, C.c_uint32, u32p]),
        "or_moddown": (None, [C.c_void_p, u32p, C.c_int, u32p]),
        "or_rotate": (None, [C.c_void_p, u32p, C.c_int, u32p, u32p, C.c_uint64, u32p]),
        "or_rotate_hoisted": (None, [C.c_void_p, u32p, C.c_int, C.c_int, u32p, C.c_void_p, u64p, C.c_void_p]),
        "or_ksk_gen": (None, [C.c_void_p, u32p, u32p, u32p, u32p, u32p]),
        "or_rotation_key": (None, [C.c_void_p, C.c_void_p, u32p, C.c_uint64, u32p, u32p]),
        "or_secret_eval": (None, [C.c_void_p, i8p, u32p]),
        "or_automorph_rows": (None, [C.c_void_p, u32p, C.c_uint32, C.c_int, u32p]),
        "or_rotate_sum": (C.c_int, [C.c_void_p, u32p, C.c_int, C.c_int, u32p, C.c_void_p, u64p, C.c_void_p, u32p]),
        "or_rotate_many": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, u32p, C.c_void_p, u64p, C.c_void_p,
                                     C.c_int, u32p]),
        "or_moddown_rescale": (None, [C.c_void_p, u32p, C.c_int, C.c_void_p, u32p]),
        "or_rotate_and_sum": (C.c_int, [C.c_void_p, u32p, C.c_int, C.c_int64, C.c_int64, C.c_int, C.c_int, u32p,
                                        C.c_void_p, u64p, u32p]),
        "or_cts_fused": (None, [C.c_void_p, C.c_int, u32p, u32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                C.c_void_p, C.c_void_p, C.c_int, u32p, C.c_void_p, C.c_int, C.c_int, C.c_uint32,
                                C.c_void_p, C.c_void_p, u32p]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


LIB = _load()


def ptr_array(arrs):
    """A C array of pointers to the numpy arrays `arrs` (kept alive by the caller)."""
    return (C.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])


def set_threads(n):
    LIB.or_set_threads(int(n))


def set_cpus(cpus):
    """pin the pool's threads one per logical CPU of the list (empty: unpinned)"""
    a = np.asarray(list(cpus) or [0], np.int32)
    LIB.or_set_cpus(a, len(cpus))


def set_kska_cache(nbytes):
    """the expanded-key cache's byte budget (0: off, cleared)"""
    LIB.or_set_kska_cache(int(nbytes))


def descending_primes(bits, m, n):
    out = np.zeros(n, np.uint64)
    if LIB.or_descending_primes(bits, m, n, out) != 0:
        raise ValueError("not enough primes")
    return [int(x) for x in out]


class Prng:
    """The sampler DRBG (ChaCha20, stream id, "DRBG" tag)."""

    def __init__(self, key, stream=0):
        self.h = LIB.or_prng_new(np.asarray(key, np.uint32), stream)

    def __del__(self):
        if getattr(self, "h", None):
            LIB.or_prng_free(self.h)

    def u32(self):
        return LIB.or_prng_next_u32(self.h)

    def u64(self):
        return LIB.or_prng_next_u64(self.h)

    def below(self, q):
        return LIB.or_prng_uniform_below(self.h, q)

    def f64(self):
        return LIB.or_prng_uniform_f64(self.h)

    def ksk_seed(self):
        s = np.zeros(8, np.uint32)
        LIB.or_prng_ksk_seed(self.h, s)
        return s

    def sparse_ternary(self, n, h):
        out = np.zeros(n, np.int8)
        if LIB.or_sample_sparse_ternary(self.h, n, h, out) != 0:
            raise ValueError("h > n")
        return out

    def gaussian(self, n, sigma=3.19):
        out = np.zeros(n, np.int64)
        LIB.or_sample_gaussian(self.h, sigma, n, out)
        return out


def below_accept(v, q):
    """uniform_below's rule on one 64-bit word: v mod q if v is accepted, else None."""
    r = C.c_uint64(0)
    return int(r.value) if LIB.or_below_accept(v, q, C.byref(r)) else None


def gauss_cdf(sigma=3.19):
    n = LIB.or_gauss_cdf(sigma, np.zeros(1, np.float64), 0)
    out = np.zeros(n, np.float64)
    LIB.or_gauss_cdf(sigma, out, n)
    return out


def gauss_index(u, sigma=3.19):
    return LIB.or_gauss_index(sigma, u)


class Ctx:
    """A chain of nq Q primes then kp special primes at N = 2^logn with dnum hybrid digits."""

    def __init__(self, logn, q, p, dnum):
        self.logn, self.n = logn, 1 << logn
        self.q, self.p = list(q), list(p)
        self.nq, self.kp, self.dnum = len(q), len(p), dnum
        self.primes = self.q + self.p
        self.rows = self.nq + self.kp
        arr = np.array(self.primes, np.uint64)
        self.h = LIB.or_ctx_new(logn, arr, self.nq, self.kp, dnum)
        if not self.h:
            raise ValueError("invalid chain")
        big_p = 1
        for x in self.p:
            big_p *= int(x)
        self.pmodq = [big_p % int(x) for x in self.q]  # P mod q_t

    def __del__(self):
        if getattr(self, "h", None):
            LIB.or_ctx_free(self.h)

    def twiddles(self, pid):
        n = self.n
        t = [np.zeros(n, np.uint32) for _ in range(4)]
        LIB.or_ctx_twiddles(self.h, pid, *t)
        return t

    def root(self, pid):
        return LIB.or_ctx_root(self.h, pid)

    def ntt_fwd(self, rows, ids):
        rows = np.ascontiguousarray(rows, np.uint32)
        LIB.or_ntt_fwd_rows(self.h, rows, np.asarray(ids, np.int32), len(ids))
        return rows

    def ntt_inv(self, rows, ids):
        rows = np.ascontiguousarray(rows, np.uint32)
        LIB.or_ntt_inv_rows(self.h, rows, np.asarray(ids, np.int32), len(ids))
        return rows

    def bconv(self, src_rows, src_ids, tgt_ids, prescaled=False):
        src = [np.ascontiguousarray(r, np.uint32) for r in src_rows]
        dst = [np.zeros(self.n, np.uint32) for _ in tgt_ids]
        LIB.or_bconv(self.h, ptr_array(src), np.asarray(src_ids, np.int32), len(src), ptr_array(dst),
                     np.asarray(tgt_ids, np.int32), len(dst), int(prescaled))
        return dst

    def live_digits(self, top):
        return LIB.or_live_digits(self.h, top)

    def digit_of(self, pid):
        return LIB.or_digit_of(self.h, pid)

    def ct_zeros(self):
        return np.zeros((2, self.rows, self.n), np.uint32)

    def modup(self, c1, top):
        digits = np.zeros((self.dnum, self.rows, self.n), np.uint32)
        LIB.or_modup(self.h, np.ascontiguousarray(c1, np.uint32), top, digits)
        return digits

    def ks_dot(self, ct, digits, top, seed, b, autok):
        ext = self.ct_zeros()
        LIB.or_ks_dot(self.h, np.ascontiguousarray(ct, np.uint32), np.ascontiguousarray(digits, np.uint32), top,
                      np.asarray(seed, np.uint32), np.ascontiguousarray(b, np.uint32), autok, ext)
        return ext

    def moddown(self, ext, top):
        out = self.ct_zeros()
        LIB.or_moddown(self.h, np.ascontiguousarray(ext, np.uint32), top, out)
        return out

    def mul_relin(self, a, b, top, seed, bkey):
        """The relinearized product (crates/pc-gpu/src/relin.rs:213-235) composed from the oracle's pieces: the tensor
        (oracle/em.py), ModUp(d2), the key dot with no c0 term and no automorphism, ModDown added onto (c0, c1)."""
        from oracle import em
        n = top + 1
        c0, c1, d2 = em.tensor(self.primes, [(a[None, :, :n], b[None, :, :n])])
        tmp = self.ct_zeros()
        tmp[1, :n] = d2[0]
        ext = self.ks_dot(tmp, self.modup(tmp[1], top), top, seed, bkey, 1)
        md = self.moddown(ext, top)
        out = self.ct_zeros()
        q = np.asarray(self.primes[:n], np.uint64).reshape(n, 1)
        out[0, :n] = ((c0[0].astype(np.uint64) + md[0, :n]) % q).astype(np.uint32)
        out[1, :n] = ((c1[0].astype(np.uint64) + md[1, :n]) % q).astype(np.uint32)
        return out

    def moddown_rescale(self, ext, top, onto=None):
        """Q rows 0..top - 2 of round((ext + P onto) / (P q_top q_{top-1})): the ModDown and the two-prime rescale as
        one exact ModDown."""
        out = self.ct_zeros()
        on = None if onto is None else np.ascontiguousarray(onto, np.uint32)
        LIB.or_moddown_rescale(self.h, np.ascontiguousarray(ext, np.uint32), top,
                               None if on is None else on.ctypes.data, out)
        return out

    def mul_relin_rescale(self, a, b, top, seed, bkey):
        """The relinearized product rescaled by the two top primes in one exact ModDown: the tensor, ModUp(d2), the key
        dot, then moddown_rescale with (d0, d1) as onto."""
        from oracle import em
        n = top + 1
        c0, c1, d2 = em.tensor(self.primes, [(a[None, :, :n], b[None, :, :n])])
        tmp = self.ct_zeros()
        tmp[1, :n] = d2[0]
        ext = self.ks_dot(tmp, self.modup(tmp[1], top), top, seed, bkey, 1)
        d = self.ct_zeros()
        d[0, :n], d[1, :n] = c0[0], c1[0]
        return self.moddown_rescale(ext, top, d)

    def mul_sum_relin_rescale(self, pairs, top, seed, bkey, add=None, sub=False, kmul=None, twice=False):
        """The sum of the pairs' tensors (a b over every pair, summed exactly mod each prime; twice: 2a b),
        relinearized and rescaled once as mul_relin_rescale does one tensor; add (a ciphertext, or None) times the
        integer kmul (None: 1) is added to the tensor's (d0, d1) first (subtracted with sub), so it is rescaled with
        the product."""
        from oracle import em
        n = top + 1
        ps = np.array(self.primes[:n], np.uint64)[:, None]
        if twice:
            pairs = [(((a[:, :n].astype(np.uint64) * 2) % ps).astype(np.uint32), b) for a, b in pairs]
        c0, c1, d2 = em.tensor(self.primes, [(a[None, :, :n], b[None, :, :n]) for a, b in pairs])
        tmp = self.ct_zeros()
        tmp[1, :n] = d2[0]
        ext = self.ks_dot(tmp, self.modup(tmp[1], top), top, seed, bkey, 1)
        d = self.ct_zeros()
        d[0, :n], d[1, :n] = c0[0], c1[0]
        if add is not None:
            km = np.array([1 if kmul is None else int(kmul) % int(p) for p in self.primes[:n]], np.uint64)[:, None]
            for part in range(2):
                x, y = d[part, :n].astype(np.uint64), add[part, :n].astype(np.uint64) * km % ps
                d[part, :n] = ((x + ps - y) if sub else (x + y)) % ps
        return self.moddown_rescale(ext, top, d)

    def rescale(self, x, top, ndrop):
        """Rows 0..top - ndrop of the rescale of one ciphertext x [2][rows][N] (oracle/em.py rescale)."""
        from oracle import em
        out = self.ct_zeros()
        out[:, : top + 1 - ndrop] = em.rescale(self, self.primes, x[None, :, : top + 1], top, ndrop)[0]
        return out

    def rotate(self, ct, top, seed, b, g):
        out = self.ct_zeros()
        LIB.or_rotate(self.h, np.ascontiguousarray(ct, np.uint32), top, np.asarray(seed, np.uint32),
                      np.ascontiguousarray(b, np.uint32), g, out)
        return out

    def rotate_hoisted(self, ct, top, seeds, bs, gs):
        outs = [self.ct_zeros() for _ in gs]
        bs = [np.ascontiguousarray(b, np.uint32) for b in bs]
        LIB.or_rotate_hoisted(self.h, np.ascontiguousarray(ct, np.uint32), top, len(gs),
                              np.ascontiguousarray(seeds, np.uint32).reshape(-1), ptr_array(bs),
                              np.asarray(gs, np.uint64), ptr_array(outs))
        return outs

    def rotate_sum(self, ct, top, seeds, bs, gs, onto=None):
        """onto + ModDown(sum of the extended rotations of ct by the keys): one ModUp, one ModDown."""
        out = self.ct_zeros()
        bs = [np.ascontiguousarray(b, np.uint32) for b in bs]
        on = None if onto is None else np.ascontiguousarray(onto, np.uint32)
        rc = LIB.or_rotate_sum(self.h, np.ascontiguousarray(ct, np.uint32), top, len(gs),
                               np.ascontiguousarray(seeds, np.uint32).reshape(-1), ptr_array(bs),
                               np.asarray(gs, np.uint64), None if on is None else on.ctypes.data, out)
        if rc:
            raise ValueError("rotate_sum: an identity key or no keys")
        return out

    def rotate_many(self, cts, top, seeds, bs, gs, onto=None, rescale=False):
        """onto + ModDown(sum of the extended rotations of cts[j] by key j): a ModUp each, one ModDown (rescale: the
        ModDown by P q_top q_{top-1}, the result at top - 2)."""
        out = self.ct_zeros()
        xs = [np.ascontiguousarray(x, np.uint32) for x in cts]
        bs = [np.ascontiguousarray(b, np.uint32) for b in bs]
        on = None if onto is None else np.ascontiguousarray(onto, np.uint32)
        rc = LIB.or_rotate_many(self.h, ptr_array(xs), top, len(gs), np.ascontiguousarray(seeds, np.uint32).reshape(-1),
                                ptr_array(bs), np.asarray(gs, np.uint64), None if on is None else on.ctypes.data,
                                int(rescale), out)
        if rc:
            raise ValueError("rotate_many: an identity key or no keys")
        return out

    def rotate_and_sum(self, x, top, start, stop, seeds, bs, gs, radix_bits=1):
        """The rotate-and-sum ladder over the keys (seeds, bs, gs)."""
        out = self.ct_zeros()
        bs = [np.ascontiguousarray(b, np.uint32) for b in bs]
        rc = LIB.or_rotate_and_sum(self.h, np.ascontiguousarray(x, np.uint32), top, start, stop, radix_bits, len(gs),
                                   np.ascontiguousarray(seeds, np.uint32).reshape(-1), ptr_array(bs),
                                   np.asarray(gs, np.uint64), out)
        if rc:
            raise ValueError("rotate_and_sum: a step's key is missing")
        return out

    def cts_fused(self, x, digits, top, B, G, pts, kinv, seeds=None, bs=(), as_=None, nregen=None, pt_prow=None,
                  enc=0xFFFFFFFF, pmod=None, x0=None):
        """The fused CtS stage of K = len(x) ciphertexts (or_cts_fused): res[c][j] = sum_i rot_i(x_c) pt_{B j + i}.
        pts: list of diagonals [prow rows][ptw]; kinv: B-1 gather exponents; seeds [B-1][8], bs / as_ [B-1] full-layout
        key rows; nregen (default: every digit) digits of a regenerated from the seed, the rest read from as_."""
        x = np.ascontiguousarray(x, np.uint32)
        K = x.shape[0]
        digits = np.ascontiguousarray(digits, np.uint32)
        nd = self.dnum if nregen is None else nregen
        bs = [np.ascontiguousarray(b, np.uint32) for b in bs]
        as_ = [np.ascontiguousarray(a, np.uint32) for a in as_] if as_ is not None else []
        pts = [np.ascontiguousarray(p, np.uint32) for p in pts]
        ptw = pts[0].shape[-1]
        res = np.zeros((K, G, 2, self.rows, self.n), np.uint32)
        sd = np.ascontiguousarray(seeds if seeds is not None else np.zeros((max(B - 1, 1), 8)), np.uint32)
        ki = np.ascontiguousarray(np.asarray(kinv, np.uint32).reshape(-1) if B > 1 else np.zeros(1), np.uint32)
        pm = None if pmod is None else np.ascontiguousarray(pmod, np.uint32)
        x0a = None if x0 is None else np.ascontiguousarray(x0, np.uint32)
        LIB.or_cts_fused(self.h, K, x, digits, top, B, G, len(pts), sd.ctypes.data, ptr_array(bs) if bs else None,
                         ptr_array(as_) if as_ else None, nd, ki, ptr_array(pts), ptw,
                         top + 1 if pt_prow is None else pt_prow, enc, None if pm is None else pm.ctypes.data,
                         None if x0a is None else x0a.ctypes.data, res)
        return res

    def ksk_gen(self, s_new, s_old, seed, e):
        b = np.zeros((self.dnum, self.rows, self.n), np.uint32)
        LIB.or_ksk_gen(self.h, np.ascontiguousarray(s_new, np.uint32), np.ascontiguousarray(s_old, np.uint32),
                       np.asarray(seed, np.uint32), np.ascontiguousarray(e, np.uint32), b)
        return b

    def rotation_key(self, prng, s_eval, g):
        seed = np.zeros(8, np.uint32)
        b = np.zeros((self.dnum, self.rows, self.n), np.uint32)
        LIB.or_rotation_key(self.h, prng.h, np.ascontiguousarray(s_eval, np.uint32), g, seed, b)
        return seed, b

    def secret_eval(self, s):
        out = np.zeros((self.rows, self.n), np.uint32)
        LIB.or_secret_eval(self.h, np.ascontiguousarray(s, np.int8), out)
        return out

    def automorph_rows(self, rows, k):
        rows = np.ascontiguousarray(rows, np.uint32)
        out = np.zeros_like(rows)
        LIB.or_automorph_rows(self.h, rows, k, rows.shape[0], out)
        return out


def kska_row(seed, digit, p, n):
    out = np.zeros(n, np.uint32)
    LIB.or_kska_expand_row(np.asarray(seed, np.uint32), digit, p, n, out)
    return out


TAG_KSKA, TAG_ENCA = 0x4B534B41, 0x454E4341


def expand_row(seed, w13, p, n, tag):
    out = np.zeros(n, np.uint32)
    LIB.or_expand_row(np.asarray(seed, np.uint32), w13, p, n, tag, out)
    return out


def cts_expand_row(seed, p, n):
    """a regenerable ciphertext's c1 row (the "CTSA" lane)"""
    out = np.zeros(n, np.uint32)
    LIB.or_cts_expand_row(np.asarray(seed, np.uint32), p, n, out)
    return out


def kskb_row(seed, digit, p, n):
    out = np.zeros(n, np.uint64)
    LIB.or_kskb_expand_row(np.asarray(seed, np.uint32), digit, p, n, out)
    return out


def chacha_block(key, w12, w13, w14, w15, rounds):
    out = np.zeros(16, np.uint32)
    LIB.or_chacha_block(np.asarray(key, np.uint32), w12, w13, w14, w15, rounds, out)
    return out


def automorph_slot(k, slot, logn):
    return LIB.or_automorph_slot(k, slot, logn)


def rotation_galois(r, n):
    return LIB.or_rotation_galois(r, n)


def galois_inverse(g, n):
    return LIB.or_galois_inverse(g, n)


def spru_fft_pass(x, tw, ns):
    """one forward Stockham pass (half-size ns) of complex128 transforms x [batch][n], twiddles tw [n/2]"""
    x = np.ascontiguousarray(x, np.complex128)
    out = np.zeros_like(x)
    LIB.or_spru_fft_pass(x.view(np.float64), out.view(np.float64),
                         np.ascontiguousarray(tw, np.complex128).view(np.float64), x.shape[-1], ns, x.shape[0])
    return out


def spru_scatter(y, zt, primes, scale):
    """coefficient rows [batch][nl][n] of complex128 FFT outputs y [batch][n] with the zeta table zt [n]"""
    y = np.ascontiguousarray(y, np.complex128)
    b, n = y.shape
    out = np.zeros((b, len(primes), n), np.uint32)
    LIB.or_spru_scatter(y.view(np.float64), np.ascontiguousarray(zt, np.complex128).view(np.float64),
                        np.array(primes, np.uint64), len(primes), n, b, scale, len(primes) * n, out)
    return out
