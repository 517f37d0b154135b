"""Host objects over the C-ABI: device buffers, streams, events, a key-switching context and key groups.

This mirrors the entry points of the reference's runtime ops (crates/pc-gpu/src/rotate.rs rotate /
rotate_hoisted, crates/pc-gpu/src/ntt.rs transform_rows, crates/pc-gpu/src/keygen.rs) with the same argument meaning;
the work itself runs in libpchip.so (the driver and the gfx950 kernels).
"""
import ctypes as C
import gc

import numpy as np

from ._lib import LIB, HipError, check
from .chains import Chain


def device_count():
    n = C.c_int(0)
    rc = LIB.pc_hip_device_count(C.byref(n))
    return n.value if rc == 0 else 0


def ntt_one_pass_min(rows):
    """Launches of N = 2^16 with at least `rows` rows take the one-pass transform (0: never); returns the previous
    threshold (pcx_ntt_one_pass_min)."""
    return int(LIB.pcx_ntt_one_pass_min(int(rows)))


class Stream:
    def __init__(self):
        self.h = C.c_void_p()
        check(LIB.pc_hip_stream_create(C.byref(self.h)), "stream_create")

    def sync(self):
        check(LIB.pc_hip_stream_sync(self.h), "stream_sync")

    def wait(self, event):
        """Later work on this stream waits for the event (recorded on another stream)."""
        check(LIB.pc_hip_stream_wait_event(self.h, event.h), "stream_wait_event")

    def __del__(self):
        if getattr(self, "h", None):
            LIB.pc_hip_stream_destroy(self.h)
            self.h = None


class Event:
    def __init__(self):
        self.h = C.c_void_p()
        check(LIB.pc_hip_event_create(C.byref(self.h)), "event_create")

    def record(self, stream):
        check(LIB.pc_hip_event_record(self.h, stream.h), "event_record")

    def sync(self):
        check(LIB.pc_hip_event_sync(self.h), "event_sync")

    def elapsed_ms(self, later):
        ms = C.c_float()
        check(LIB.pc_hip_event_elapsed_ms(C.byref(ms), self.h, later.h), "event_elapsed")
        return ms.value

    def __del__(self):
        if getattr(self, "h", None):
            LIB.pc_hip_event_destroy(self.h)
            self.h = None


class Graph:
    """A HIP graph of the work fn() enqueues on `stream` (stream capture; the launchers and the driver are capture
    safe: they never allocate, synchronise or read device data on the host), replayed by launch(). Launch-bound
    sequences of small kernels (a ladder of single key switches at a few limbs) pay their launch costs once."""

    def __init__(self, stream, fn):
        self.graph, self.exe = C.c_void_p(), C.c_void_p()
        # no device memory may be freed while the stream is captured (a free invalidates the capture): a DevBuf whose
        # last reference sits in a reference cycle (a buffer pool's replaced buffer held by an earlier run's closures)
        # is freed by the cyclic collector whenever it runs, so collect now and hold the collector off until the
        # capture has ended
        gc.collect()
        was = gc.isenabled()
        gc.disable()
        try:
            check(LIB.pc_hip_graph_begin_capture(stream.h), "graph_begin_capture")
            try:
                fn()
            finally:
                rc = LIB.pc_hip_graph_end_capture(stream.h, C.byref(self.graph))
        finally:
            if was:
                gc.enable()
        check(rc, "graph_end_capture")
        check(LIB.pc_hip_graph_instantiate(C.byref(self.exe), self.graph), "graph_instantiate")

    def launch(self, stream):
        check(LIB.pc_hip_graph_launch(self.exe, stream.h), "graph_launch")

    def __del__(self):
        if getattr(self, "exe", None) and self.exe.value:
            LIB.pc_hip_graph_exec_destroy(self.exe)
            self.exe = None
        if getattr(self, "graph", None) and self.graph.value:
            LIB.pc_hip_graph_destroy(self.graph)
            self.graph = None


class DevBuf:
    """A device allocation of u32 words."""

    def __init__(self, words):
        self.words = int(words)
        self.ptr = C.c_void_p()
        check(LIB.pc_hip_malloc(C.byref(self.ptr), max(4 * self.words, 16)), "malloc")

    @classmethod
    def from_array(cls, a, stream=None):
        a = np.ascontiguousarray(a, dtype=np.uint32)
        b = cls(a.size)
        b.upload(a, stream)
        return b

    def upload(self, a, stream=None, offset=0):
        a = np.ascontiguousarray(a, dtype=np.uint32)
        assert offset + a.size <= self.words
        s = stream.h if stream else None
        check(LIB.pc_hip_memcpy_htod(self.addr(offset), a.ctypes.data, 4 * a.size, s), "htod")
        if stream:
            stream.sync()
        else:
            check(LIB.pc_hip_device_sync(), "sync")

    def download(self, shape=None, stream=None, offset=0, words=None):
        words = self.words - offset if words is None else words
        out = np.empty(words, np.uint32)
        s = stream.h if stream else None
        check(LIB.pc_hip_memcpy_dtoh(out.ctypes.data, self.addr(offset), 4 * words, s), "dtoh")
        if stream:
            stream.sync()
        else:
            check(LIB.pc_hip_device_sync(), "sync")
        return out.reshape(shape) if shape is not None else out

    def zero(self):
        check(LIB.pc_hip_memset(self.ptr, 0, 4 * self.words, None), "memset")
        check(LIB.pc_hip_device_sync(), "sync")

    def addr(self, offset=0):
        return C.c_void_p(self.ptr.value + 4 * int(offset))

    def __del__(self):
        if getattr(self, "ptr", None) and self.ptr.value:
            LIB.pc_hip_free(self.ptr)
            self.ptr = None


def _u64(xs):
    return (C.c_uint64 * len(xs))(*[int(x) for x in xs])


class Context:
    """One chain on the device: tables, per-top plans and a workspace for k_rot extended ciphertexts; k_max: the
    ciphertexts a batched product or rescale takes (pcx_ctx_new_k)."""

    def __init__(self, chain: Chain, k_rot=1, k_max=1):
        self.chain = chain
        self.n, self.logn = chain.n, chain.logn
        self.nq, self.kp, self.dnum, self.rows = len(chain.q), len(chain.p), chain.dnum, chain.rows
        if self.kp < 1:
            raise ValueError("a key-switching context needs at least one special prime")
        err = C.c_int(0)
        self.h = LIB.pcx_ctx_new_k(chain.logn, _u64(chain.primes), self.nq, self.kp, chain.dnum, k_rot, k_max,
                                   C.byref(err))
        if not self.h:
            raise HipError(f"pcx_ctx_new_k failed: {err.value}")
        self.k_rot, self.k_max = k_rot, k_max
        self.ct_words = 2 * self.rows * self.n

    def __del__(self):
        if getattr(self, "h", None):
            LIB.pcx_ctx_free(self.h)
            self.h = None

    def ct_buf(self, count=1):
        return DevBuf(count * self.ct_words)

    def conv_fusion(self, mask=-1):
        """The conversions streamed into the NTT column pass (pcx_ctx_conv_fusion: bit 0 ModUp, 1 ModDown, 2 the
        ModDown-rescale); mask < 0 only reads. Returns the previous mask."""
        return int(LIB.pcx_ctx_conv_fusion(self.h, int(mask)))

    def table_only(self, on=True):
        """Issue every operation through the kernel table alone (pcx_ctx_table_only); returns the previous setting."""
        return bool(LIB.pcx_ctx_table_only(self.h, int(on)))

    def modup(self, ct, top, stream):
        check(LIB.pcx_modup(self.h, ct.addr(), top, stream.h), "modup")

    def modup_digits(self, stream):
        """The ModUp workspace [dnum][rows][N] (a copy)."""
        stream.sync()
        p = LIB.pcx_modup_digits(self.h)
        out = np.empty(self.dnum * self.rows * self.n, np.uint32)
        check(LIB.pc_hip_memcpy_dtoh(out.ctypes.data, p, out.nbytes, stream.h), "dtoh")
        stream.sync()
        return out.reshape(self.dnum, self.rows, self.n)

    def dot(self, keys, r, ct, top, ext, stream):
        check(LIB.pcx_dot(self.h, keys.h, r, ct.addr(), top, ext.addr(), stream.h), "dot")

    def moddown(self, ext, top, out, stream):
        check(LIB.pcx_moddown(self.h, ext.addr(), top, out.addr(), stream.h), "moddown")

    STAGES = ("modup_intt", "modup_bconv", "modup_ntt", "dot", "md_intt", "md_bconv", "md_ntt", "cts", "tensor",
              "rescale")

    def timing(self, max_stages):
        """Record device time per stage (0 turns it off)."""
        check(LIB.pcx_timing(self.h, max_stages), "timing")

    def timing_read(self):
        """{stage: (total ms, launches)} of the stages recorded since timing() (after a sync)."""
        out = {}
        for i, name in enumerate(self.STAGES):
            ms, n = C.c_double(), C.c_int()
            check(LIB.pcx_timing_read(self.h, i, C.byref(ms), C.byref(n)), "timing_read")
            out[name] = (ms.value, n.value)
        return out

    def rotate(self, keys, r, ct, top, out, stream):
        check(LIB.pcx_rotate(self.h, keys.h, r, ct.addr(), top, out.addr(), stream.h), "rotate")

    def rotate_hoisted(self, keys, idx, ct, top, out, stream):
        arr = (C.c_int * len(idx))(*idx)
        check(LIB.pcx_rotate_hoisted(self.h, keys.h, arr, len(idx), ct.addr(), top, out.addr(), stream.h),
              "rotate_hoisted")

    def rotate_sum(self, keys, idx, ct, top, out, stream, onto=None):
        """out = onto + sum_j rot(ct, key idx[j]): one ModUp, the dots summed, one ModDown (pcx_rotate_sum)."""
        arr = (C.c_int * len(idx))(*idx)
        check(LIB.pcx_rotate_sum(self.h, keys.h, arr, len(idx), ct.addr(), top, out.addr(),
                                 None if onto is None else onto.addr(), stream.h), "rotate_sum")

    def rotate_many(self, keys, idx, cts, top, out, stream, onto=None):
        """out = onto + sum_j rot(cts[j], key idx[j]): a ModUp and a key dot per input, the dots summed in the
        extended basis, one ModDown (pcx_rotate_many)."""
        arr = (C.c_int * len(idx))(*idx)
        ptrs = (C.c_void_p * len(cts))(*[x.addr() for x in cts])
        check(LIB.pcx_rotate_many(self.h, keys.h, arr, len(idx), ptrs, top, out.addr(),
                                  None if onto is None else onto.addr(), stream.h), "rotate_many")

    def rotate_many_rescale(self, keys, idx, cts, top, out, stream, onto=None):
        """rotate_many with the two-prime rescale fused into its ModDown: out at top - 2 (pcx_rotate_many_rescale)."""
        arr = (C.c_int * len(idx))(*idx)
        ptrs = (C.c_void_p * len(cts))(*[x.addr() for x in cts])
        check(LIB.pcx_rotate_many_rescale(self.h, keys.h, arr, len(idx), ptrs, top, out.addr(),
                                          None if onto is None else onto.addr(), stream.h), "rotate_many_rescale")

    def rotate_and_sum(self, keys, x, top, start, stop, out, tmp, stream, radix_bits=1, K=1):
        """The rotate-and-sum ladder: out = sum of x over its rotations by the multiples of start below stop; K > 1: K
        consecutive ciphertexts rung by rung together (pcx_rotate_and_sum_k)."""
        if K == 1:
            check(LIB.pcx_rotate_and_sum(self.h, keys.h, x.addr(), top, start, stop, radix_bits, out.addr(),
                                         tmp.addr(), stream.h), "rotate_and_sum")
        else:
            check(LIB.pcx_rotate_and_sum_k(self.h, keys.h, x.addr(), top, start, stop, radix_bits, out.addr(),
                                           tmp.addr(), K, stream.h), "rotate_and_sum_k")

    def rescale(self, ct, top, ndrop, out, stream, K=1):
        """out's rows 0..top - ndrop = the rescale of ct by its top ndrop (1 or 2) primes (pcx_rescale); K > 1: K
        consecutive ciphertexts in the same launches (pcx_rescale_k)."""
        if K == 1:
            check(LIB.pcx_rescale(self.h, ct.addr(), top, ndrop, out.addr(), stream.h), "rescale")
        else:
            check(LIB.pcx_rescale_k(self.h, ct.addr(), top, ndrop, out.addr(), K, stream.h), "rescale_k")

    def mul_plain(self, ct, pt, top, out, stream):
        """out = ct pt on Q rows 0..top (pcx_mul_plain); pt a DevBuf of evaluation-form rows by prime id."""
        check(LIB.pcx_mul_plain(self.h, ct.addr(), pt.addr(), top, out.addr(), stream.h), "mul_plain")

    def mul_plain_k(self, ct, pts, top, out, stream):
        """ct and out each len(pts) consecutive ciphertexts: out_j = ct_j pts[j] in one launch (pcx_mul_plain_k)."""
        arr = (C.c_void_p * len(pts))(*[p.addr() for p in pts])
        check(LIB.pcx_mul_plain_k(self.h, ct.addr(), arr, len(pts), top, out.addr(), stream.h), "mul_plain_k")

    def mul_relin(self, keys, a, b, top, out, stream):
        """out = a b relinearized by key 0 of keys (pcx_mul_relin)."""
        check(LIB.pcx_mul_relin(self.h, keys.h, a.addr(), b.addr(), top, out.addr(), stream.h), "mul_relin")

    def mul_relin_rescale(self, keys, a, b, top, out, stream, K=1, twice=False):
        """out (top - 2) = a b relinearized and rescaled by the two top primes in one ModDown (pcx_mul_relin_rescale);
        K > 1: K consecutive pairs in the same launches, twice: 2 a b (pcx_mul_relin_rescale_k)."""
        if K == 1 and not twice:
            check(LIB.pcx_mul_relin_rescale(self.h, keys.h, a.addr(), b.addr(), top, out.addr(), stream.h),
                  "mul_relin_rescale")
        else:
            check(LIB.pcx_mul_relin_rescale_k(self.h, keys.h, a.addr(), b.addr(), top, out.addr(), K, int(twice),
                                              stream.h), "mul_relin_rescale_k")

    def mul_relin_rescale_list(self, keys, a, b, top, out, stream, twice=False):
        """out's len(a) consecutive ciphertexts (top - 2) = a[j] b[j] relinearized and rescaled, the pairs at their own
        addresses: one tensor launch for all, then the batched ModUp, dots and ModDown (pcx_mul_relin_rescale_list)."""
        assert len(a) == len(b) >= 1
        pa = (C.c_void_p * len(a))(*[x.addr() for x in a])
        pb = (C.c_void_p * len(b))(*[x.addr() for x in b])
        check(LIB.pcx_mul_relin_rescale_list(self.h, keys.h, pa, pb, len(a), top, out.addr(), int(twice), stream.h),
              "mul_relin_rescale_list")

    def mul_sum_relin_rescale_list(self, keys, groups, top, out, stream, adds=None, sub=0, kmuls=None, twice=False):
        """out's len(groups) consecutive ciphertexts (top - 2): product j = the sum of a b over the pairs (a, b) of
        groups[j] (doubled with twice) plus adds[j] times kmuls[j] (a ciphertext at top or above whose multiple sits
        at the products' scale, or None; the multiplier a DevBuf of the rows' k mod q then Shoup companions, or None
        for 1; subtracted where bit j of sub is set), relinearized and rescaled once
        (pcx_mul_sum_relin_rescale_list)."""
        pairs = [p for g in groups for p in g]
        assert groups and all(groups)
        assert adds is None or len(adds) == len(groups)
        off = [0]
        for g in groups:
            off.append(off[-1] + len(g))
        pa = (C.c_void_p * len(pairs))(*[x.addr() for x, _ in pairs])
        pb = (C.c_void_p * len(pairs))(*[y.addr() for _, y in pairs])
        po = (C.c_int * len(off))(*off)
        py = None if adds is None else (C.c_void_p * len(adds))(*[None if y is None else y.addr() for y in adds])
        pk = None if kmuls is None else (C.c_void_p * len(kmuls))(*[None if k is None else k.addr() for k in kmuls])
        check(LIB.pcx_mul_sum_relin_rescale_list(self.h, keys.h, pa, pb, po, len(groups), top, py, pk, int(sub),
                                                 1 if twice else 0, out.addr(), stream.h), "mul_sum_relin_rescale_list")

    def cts_stage(self, keys, r0, B, G, pts, npts, ptw, enc, ct, top, res, stream):
        """One CtS / StC stage's baby steps and plaintext products (pcx_cts_stage): res_j = sum_i rot_i(ct) pt_{Bj+i}
        in the extended basis, babies i >= 1 by keys r0 + i - 1. pts: a DevBuf holding npts device pointers (uint64)
        to the diagonals [top + 1 + kp rows][ptw]; res: G extended ciphertexts."""
        check(LIB.pcx_cts_stage(self.h, keys.h, r0, B, G, pts.addr(), npts, ptw, enc, ct.addr(), top, res.addr(),
                                stream.h), "cts_stage")

    def cts_stage_hoisted(self, keys, r0, B, G, pts, npts, ptw, enc, ct, top, rot, res, stream):
        """cts_stage's words by the hoisted route (pcx_cts_stage_hoisted): rot_0 = P ct, one ModUp and one key-dot
        launch for the babies into rot's B extended ciphertexts, then the plaintext dot over the extended rows."""
        check(LIB.pcx_cts_stage_hoisted(self.h, keys.h, r0, B, G, pts.addr(), npts, ptw, enc, ct.addr(), top,
                                        rot.addr(), res.addr(), stream.h), "cts_stage_hoisted")

    def moddown_k(self, ext, top, out, m, stream):
        """ModDown of m extended ciphertexts into m ciphertexts, one launch sequence (pcx_moddown_k)"""
        check(LIB.pcx_moddown_k(self.h, ext.addr(), top, out.addr(), m, stream.h), "moddown_k")


def band_digits(ctx, q_top):
    """the digits a key banded at q_top stores: every digit whose first prime id is <= q_top"""
    alpha = -(-ctx.nq // ctx.dnum)
    return q_top // alpha + 1


def band_rows(b, ctx, q_top):
    """a full key's b [dnum][nq + kp][N] restricted to the band at q_top: digits 0..ndig, rows 0..=q_top then P"""
    b = np.asarray(b)
    nd = band_digits(ctx, q_top)
    return np.ascontiguousarray(np.concatenate([b[:nd, : q_top + 1], b[:nd, ctx.nq:]], axis=1))


class Drbg:
    """The key-generation sampler's DRBG on the host (pcx_drbg_*: crates/pc-core/src/keys.rs:113-325 Prng with its
    sparse ternary and discrete Gaussian samplers)."""

    def __init__(self, key, stream=0):
        k = np.ascontiguousarray(key, np.uint32).reshape(8)
        self.h = LIB.pcx_drbg_new(k.ctypes.data_as(C.POINTER(C.c_uint32)), int(stream))
        if not self.h:
            raise HipError("pcx_drbg_new failed")

    def u32(self):
        return int(LIB.pcx_drbg_u32(self.h))

    def ksk_seed(self):
        out = np.zeros(8, np.uint32)
        check(LIB.pcx_drbg_ksk_seed(self.h, out.ctypes.data_as(C.POINTER(C.c_uint32))), "drbg_ksk_seed")
        return out

    def sparse_ternary(self, n, h):
        out = np.zeros(n, np.int8)
        if LIB.pcx_drbg_sparse_ternary(self.h, n, h, out.ctypes.data_as(C.POINTER(C.c_int8))) != 0:
            raise ValueError(f"sparse ternary: h={h} > n={n}")
        return out

    def gaussian(self, n, sigma=3.19):
        out = np.zeros(n, np.int64)
        check(LIB.pcx_drbg_gaussian(self.h, sigma, n, out.ctypes.data_as(C.POINTER(C.c_int64))), "drbg_gaussian")
        return out

    def keygen_draw(self, nkeys, ndig, n, sigma=3.19):
        """(seeds[nkeys][8], errors[nkeys][ndig][n]) in crates/pc-gpu/src/keygen.rs:193-210 order (pcx_keygen_draw)"""
        seeds = np.zeros((nkeys, 8), np.uint32)
        errors = np.zeros((nkeys, ndig, n), np.int64)
        check(LIB.pcx_keygen_draw(self.h, nkeys, ndig, n, sigma, seeds.ctypes.data_as(C.POINTER(C.c_uint32)),
                                  errors.ctypes.data_as(C.POINTER(C.c_int64))), "keygen_draw")
        return seeds, errors

    def __del__(self):
        if getattr(self, "h", None):
            LIB.pcx_drbg_free(self.h)
            self.h = None


class Keys:
    """A key group: rotation keys by galois element, a regenerated from each seed, b stored dense or packed. relin:
    the relinearization key s^2 -> s (galois 1, generated from secret / errors)."""

    def __init__(self, ctx: Context, galois, seeds=None, b=None, bits=0, secret=None, errors=None, relin=False,
                 q_top=None):
        """q_top: a banded group (host b given as [ndig][q_top + 1 + kp][N] per key, pcx_keys_new_banded)"""
        self.ctx = ctx
        self.galois = [int(g) for g in galois]
        n = len(self.galois)
        err = C.c_int(0)
        seeds = np.ascontiguousarray(seeds, np.uint32).reshape(n, 8)
        sp = seeds.ctypes.data_as(C.POINTER(C.c_uint32))
        self._keep = [seeds]
        if relin:
            if self.galois != [1] or secret is None:
                raise ValueError("the relinearization key is one key of galois 1 generated from the secret")
            s = np.ascontiguousarray(secret, np.int8)
            e = np.ascontiguousarray(errors, np.int64).reshape(1, ctx.dnum, ctx.n)
            self._keep += [s, e]
            self.h = LIB.pcx_keys_relin(ctx.h, s.ctypes.data_as(C.POINTER(C.c_int8)), sp,
                                        e.ctypes.data_as(C.POINTER(C.c_int64)), bits, C.byref(err))
        elif b is not None:
            bs = [np.ascontiguousarray(x, np.uint32) for x in b]
            self._keep += bs
            ptrs = (C.c_void_p * n)(*[x.ctypes.data for x in bs])
            if q_top is None:
                self.h = LIB.pcx_keys_new(ctx.h, n, _u64(self.galois), sp, ptrs, bits, C.byref(err))
            else:
                self.h = LIB.pcx_keys_new_banded(ctx.h, n, _u64(self.galois), sp, ptrs, bits, int(q_top),
                                                 C.byref(err))
        else:
            s = np.ascontiguousarray(secret, np.int8)
            e = np.ascontiguousarray(errors, np.int64).reshape(n, ctx.dnum, ctx.n)
            self._keep += [s, e]
            self.h = LIB.pcx_keys_generate(ctx.h, n, _u64(self.galois), s.ctypes.data_as(C.POINTER(C.c_int8)), sp,
                                           e.ctypes.data_as(C.POINTER(C.c_int64)), bits, C.byref(err))
        if not self.h:
            raise HipError(f"key group failed: {err.value}")
        self._keep = None
        self.bits = bits

    def resident_a(self, regen_digits, stream):
        """Store every key's `a` on the device and regenerate only digits < regen_digits (pcx_keys_resident_a)."""
        check(LIB.pcx_keys_resident_a(self.h, int(regen_digits), stream.h), "keys_resident_a")

    def resident_bytes(self):
        return int(LIB.pcx_keys_resident_bytes(self.h))

    def patch_bytes(self):
        """Bytes of the group's KSKA retry-value table (0 when the dot redraws in the kernel)."""
        return int(LIB.pcx_keys_patch_bytes(self.h))

    def q_top(self):
        """the highest ciphertext top the group serves"""
        return int(LIB.pcx_keys_q_top(self.h))

    def download_b(self, r):
        qt = self.q_top()
        if qt == self.ctx.nq - 1:
            shape = (self.ctx.dnum, self.ctx.rows, self.ctx.n)
        else:
            shape = (band_digits(self.ctx, qt), qt + 1 + self.ctx.kp, self.ctx.n)
        out = np.empty(shape, np.uint32)
        check(LIB.pcx_keys_download_b(self.h, r, out.ctypes.data_as(C.POINTER(C.c_uint32))), "download_b")
        return out

    def __del__(self):
        if getattr(self, "h", None):
            LIB.pcx_keys_free(self.h)
            self.h = None


class Rows:
    """A device row list for batched transforms: row i at base + roff[i] N, prime id ids[i]."""

    def __init__(self, ctx, roff, ids):
        self.ctx = ctx
        ro = np.ascontiguousarray(roff, np.uint32)
        ii = np.ascontiguousarray(ids, np.int32)
        self.n = len(ro)
        self.h = LIB.pcx_rows_new(ctx.h, ro.ctypes.data_as(C.POINTER(C.c_uint32)),
                                  ii.ctypes.data_as(C.POINTER(C.c_int32)), self.n)
        if not self.h:
            raise HipError("pcx_rows_new failed")

    def ntt(self, base, direction, stream):
        check(LIB.pcx_ntt(self.ctx.h, direction, base.addr(), self.h, stream.h), "ntt")

    def __del__(self):
        if getattr(self, "h", None):
            LIB.pcx_rows_free(self.h)
            self.h = None


class Decryptor:
    """Decryption on the device (pcx_decryptor, crates/pc-gpu/src/decrypt.rs): c0 + c1 s over the bottom d rows of
    each ciphertext, then the inverse NTT; coefficient rows out."""

    def __init__(self, ctx, d, k_max=1):
        self.ctx, self.d, self.k_max = ctx, int(d), int(k_max)
        err = C.c_int(0)
        self.h = LIB.pcx_decryptor_new(ctx.h, self.d, self.k_max, C.byref(err))
        if not self.h:
            raise HipError(f"pcx_decryptor_new: {err.value}")
        self.out = DevBuf(self.k_max * self.d * ctx.chain.n)

    def load_secret(self, s_rows, stream):
        """s_rows: the secret's evaluation-form rows [nwhich][d][N] (dense, then sparse)."""
        s = np.ascontiguousarray(s_rows, np.uint32)
        s = s.reshape(-1, self.d, self.ctx.chain.n)
        check(LIB.pcx_decryptor_load_secret(self.h, s.ctypes.data_as(C.POINTER(C.c_uint32)), s.shape[0],
                                            stream.h), "decryptor_load_secret")

    def decrypt_rows(self, ct, top, stream, K=1, which=0):
        """[K][d][N] coefficient rows of K consecutive ciphertexts at top (synchronises stream)."""
        check(LIB.pcx_decrypt_rows(self.h, ct.addr(), K, top, which, self.out.ptr, stream.h), "decrypt_rows")
        stream.sync()
        return self.out.download((K, self.d, self.ctx.chain.n), stream=stream, words=K * self.d * self.ctx.chain.n)

    def __del__(self):
        if getattr(self, "h", None):
            LIB.pcx_decryptor_free(self.h)
            self.h = None
