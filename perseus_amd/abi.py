"""ctypes mirrors of the ABI-30 argument structs a Python caller fills to call the kernel table's entries directly
(include/pc_hip.h; the reference's crates/pc-kernels/src/args.rs mirrors the same C structs field for field), and the
table's entries by name in args.cuh's order (args.cuh:1037-1097)."""
import ctypes as C

from ._lib import LIB

vp = C.c_void_p
i32, u32, u64 = C.c_int32, C.c_uint32, C.c_uint64

# the 52 launchers of KernelTable, in table order
ENTRIES = (
    "ntt_fwd ntt_inv bconv ew_add ew_scale ew_sub_mul ew_copy pt_dot ks_dot ks_dot_regen ksk_expand cts_fused tensor "
    "md_epilogue wsum add_const mul_table rescale_coef rescale_combine automorph encode encrypt ksk_gen ksk_unpack "
    "mod_raise small_int spru_extract spru_fft_pass spru_scatter cts_fused_regen ks_dot_key pcmm ccmm wsum_k "
    "rescale_combine_to md_epilogue_to small_int1 coeff_sum mul_add rescale_fwd mul_add_n tensor_y wsum_multi "
    "bconv_wide tfhe tensor_sum tensor_multi tensor_seeded ew_many submul_many pack_split pack_dot").split()
assert len(ENTRIES) == 52


class KeyTab(C.Structure):
    """args.cuh:279-290: a key set read in its stored form (40 bytes)."""
    _fields_ = [("kb", vp), ("seed", vp), ("row_words", u64), ("bits", i32), ("q_top", i32), ("srows", i32),
                ("nregen", i32)]


class CtsArgs(C.Structure):
    """args.cuh:325-355: the fused CtS stage core (200 bytes)."""
    _fields_ = [("x", vp), ("modup", vp), ("res", vp), ("kb", vp), ("ka", vp), ("kinv", vp), ("pts", vp),
                ("rows", vp), ("digit_of", vp), ("pmod", vp), ("pmods", vp), ("pr", vp), ("ct_stride", u64),
                ("part_stride", u64), ("mu_ct_stride", u64), ("mu_digit_stride", u64), ("key_digit_stride", u64),
                ("K", i32), ("B", i32), ("G", i32), ("npts", i32), ("ndig", i32), ("nq", i32), ("nlive", i32),
                ("ptw", i32), ("pt_prow", i32), ("enc", u32), ("ngrp", i32), ("nrows", i32), ("kmax", i32),
                ("pair_cts", i32), ("x0", vp)]


class CtsRegenArgs(C.Structure):
    """args.cuh:748-758: cts_fused with the baby keys through a KeyTab (240 bytes)."""
    _fields_ = [("cts", CtsArgs), ("key", KeyTab)]


class KsArgs(C.Structure):
    """args.cuh:211-228: the key-switch inner product (176 bytes)."""
    _fields_ = [("c1", vp), ("modup", vp), ("c0", vp), ("out0", vp), ("out1", vp), ("kb", vp), ("ka", vp),
                ("autok", vp), ("rows", vp), ("digit_of", vp), ("pmod", vp), ("pmods", vp), ("pr", vp),
                ("ct_stride", u64), ("mu_ct_stride", u64), ("mu_digit_stride", u64), ("out_ct_stride", u64),
                ("out_rot_stride", u64), ("key_digit_stride", u64), ("K", i32), ("R", i32), ("ndig", i32),
                ("c0_mode", i32), ("nq", i32), ("nrows", i32)]


class KsKeyArgs(C.Structure):
    """args.cuh:760-768: ks_dot with the keys through a KeyTab (216 bytes)."""
    _fields_ = [("ks", KsArgs), ("key", KeyTab)]


class EpiArgs(C.Structure):
    """args.cuh:263-277: the fused relinearisation epilogue (72 bytes)."""
    _fields_ = [("dst", vp), ("conv", vp), ("binv", vp), ("binvs", vp), ("k", vp), ("part_stride", u64),
                ("dbl", i32), ("pad", i32), ("alpha", vp), ("alphas", vp)]


class KsRegenArgs(C.Structure):
    """args.cuh:292-304: the relinearisation dot with a regenerated key (312 bytes)."""
    _fields_ = [("ks", KsArgs), ("seed", vp), ("epi", EpiArgs), ("use_epi", i32), ("pad", i32), ("key", KeyTab),
                ("add", vp)]


class PolyRef(C.Structure):
    """args.cuh:59-64: a ciphertext buffer: ct c part k row r at base + c ct_stride + k part_stride + r N words."""
    _fields_ = [("base", vp), ("ct_stride", u64), ("part_stride", u64)]


class NttArgs(C.Structure):
    """args.cuh:67-107 (176 bytes)."""
    _fields_ = [("base", vp), ("roff", vp), ("rprime", vp), ("fw", vp), ("fws", vp), ("iw", vp), ("iws", vp),
                ("ninv", vp), ("ninvs", vp), ("pr", vp), ("nrows", i32), ("chunk", i32), ("src", vp), ("soff", vp),
                ("eout", vp), ("ex", vp), ("es", vp), ("ess", vp), ("epi", i32), ("snum", i32), ("sstride", u64),
                ("xnum", i32), ("lazy", i32), ("xstride", u64), ("ed", vp)]


class RowSet(C.Structure):
    """args.cuh:52-57: Q rows [0, nq) then np special rows from prime id qmax."""
    _fields_ = [("nq", i32), ("np", i32), ("qmax", i32), ("pad", i32)]


COEFF_MAXT = 32


class CoeffArgs(C.Structure):
    """args.cuh:906-927 (592 bytes): coeff_sum."""
    _fields_ = [("scratch", vp), ("out", vp), ("fw", vp), ("fws", vp), ("pr", vp), ("overflow", vp),
                ("part_stride", u64), ("scale", C.c_double), ("n", i32), ("L", i32), ("accumulate", i32),
                ("pad", i32), ("rows", vp * COEFF_MAXT), ("ct", vp * COEFF_MAXT)]


class SpruFftArgs(C.Structure):
    """args.cuh:726-734 (32 bytes): spru_fft_pass."""
    _fields_ = [("inp", vp), ("out", vp), ("tw", vp), ("ns", i32), ("batch", i32)]


class SpruScatterArgs(C.Structure):
    """args.cuh:735-746 (56 bytes): spru_scatter."""
    _fields_ = [("y", vp), ("out", vp), ("zt", vp), ("pr", vp), ("scale", C.c_double), ("nl", i32), ("batch", i32),
                ("out_stride", u64)]


TSEED_OUT, TSEED_PAIRS, TSEED_Q, TSEED_QOUT = 16, 128, 4, 64


class TensorSeededArgs(C.Structure):
    """args.cuh:407-436 (25656 bytes): tensor_seeded."""
    _fields_ = [("out", PolyRef * TSEED_QOUT), ("d2", PolyRef * TSEED_QOUT), ("b", PolyRef * TSEED_PAIRS),
                ("a", (vp * TSEED_PAIRS) * TSEED_OUT), ("pr", vp), ("seed_off", u64), ("nout", i32), ("npairs", i32),
                ("acc", i32), ("n", i32), ("packed", i32), ("pad", i32), ("bq", (vp * TSEED_PAIRS) * (TSEED_Q - 1)),
                ("nq", i32), ("cout", i32), ("swords", i32), ("qpad", i32)]


class EwArgs(C.Structure):
    """args.cuh:144-157 (128 bytes): element-wise row-set kernels (ew_add / ew_scale / ew_sub_mul / ew_copy)."""
    _fields_ = [("out", PolyRef), ("a", PolyRef), ("b", PolyRef), ("rs", RowSet), ("sc", vp), ("scs", vp),
                ("pr", vp), ("K", i32), ("nparts", i32), ("sub", i32), ("zero_p", i32)]


class PtDotArgs(C.Structure):
    """args.cuh:184-198 (128 bytes)."""
    _fields_ = [("rot", PolyRef), ("res", PolyRef), ("rot_stride", u64), ("res_stride", u64), ("pts", vp), ("pr", vp),
                ("rs", RowSet), ("npts", i32), ("bstep", i32), ("gstep", i32), ("K", i32), ("ptw", i32),
                ("pt_prow", i32), ("enc", u32), ("pad", i32)]


class PackSplitArgs(C.Structure):
    """args.cuh:230-241 (64 bytes)."""
    _fields_ = [("q", vp), ("p", vp), ("out", vp), ("q_stride", u64), ("p_stride", u64), ("out_stride", u64),
                ("K", i32), ("sub", i32), ("nq", i32), ("nrows", i32)]


class PackDotArgs(C.Structure):
    """args.cuh:243-259 (120 bytes)."""
    _fields_ = [("dig", vp), ("kb", vp), ("ka", vp), ("c0", vp), ("out0", vp), ("out1", vp), ("rows", vp),
                ("pmod", vp), ("pmods", vp), ("pr", vp), ("dig_stride", u64), ("ct_stride", u64),
                ("out_ct_stride", u64), ("K", i32), ("sub", i32), ("nq", i32), ("nrows", i32)]


class TensorArgs(C.Structure):
    """args.cuh:356-367 (192 bytes)."""
    _fields_ = [("out", PolyRef), ("d2", PolyRef), ("a0", PolyRef), ("b0", PolyRef), ("a1", PolyRef),
                ("b1", PolyRef), ("coef", vp), ("coef_ct_stride", u64), ("pr", vp), ("npairs", i32), ("acc", i32),
                ("n", i32), ("K", i32), ("dbl", i32), ("acc_d2", i32)]


class TensorYArgs(C.Structure):
    """args.cuh:369-378 (240 bytes)."""
    _fields_ = [("t", TensorArgs), ("y", PolyRef), ("c", vp), ("cs", vp), ("sub", i32), ("pad", i32)]


TSUM_MAX = 16


class TensorSumArgs(C.Structure):
    """args.cuh:379-389."""
    _fields_ = [("out", PolyRef), ("d2", PolyRef), ("a", PolyRef * TSUM_MAX), ("b", PolyRef * TSUM_MAX), ("pr", vp),
                ("npairs", i32), ("acc", i32), ("n", i32), ("K", i32)]


TMULTI_OUT, TMULTI_PAIRS = 4, 32


class TensorMultiArgs(C.Structure):
    """args.cuh:391-406."""
    _fields_ = [("out", PolyRef * TMULTI_OUT), ("d2", PolyRef * TMULTI_OUT),
                ("a", (PolyRef * TMULTI_PAIRS) * TMULTI_OUT), ("b", (PolyRef * TMULTI_PAIRS) * TMULTI_OUT),
                ("pr", vp), ("nout", i32), ("npairs", i32), ("acc", i32), ("n", i32), ("K", i32), ("pad", i32)]


class MdEpiArgs(C.Structure):
    """args.cuh:438-447 (120 bytes)."""
    _fields_ = [("dst", PolyRef), ("x", PolyRef), ("t", PolyRef), ("binv", vp), ("binvs", vp), ("k", vp),
                ("pr", vp), ("dbl", i32), ("n", i32), ("K", i32), ("pad", i32)]


class MdEpiToArgs(C.Structure):
    """args.cuh:449-456 (152 bytes)."""
    _fields_ = [("m", MdEpiArgs), ("a", PolyRef), ("sub", i32), ("pad", i32)]


class WsumArgs(C.Structure):
    """args.cuh:458-467 (256 bytes)."""
    _fields_ = [("out", PolyRef), ("src", PolyRef * 8), ("w", vp), ("ws", vp), ("pr", vp), ("nsrc", i32),
                ("rowstride", i32), ("n", i32), ("K", i32)]


class WsumKArgs(C.Structure):
    """args.cuh:469-474 (264 bytes)."""
    _fields_ = [("w", WsumArgs), ("k", vp)]


class WsumMultiArgs(C.Structure):
    """args.cuh:476-489 (376 bytes)."""
    _fields_ = [("out", PolyRef * 3), ("src", PolyRef * 8), ("w", vp * 3), ("ws", vp * 3), ("k", vp * 3), ("pr", vp),
                ("nout", i32), ("nsrc", i32), ("rowstride", i32), ("K", i32), ("n", i32 * 3), ("nmax", i32)]


class AddConstArgs(C.Structure):
    """args.cuh:491-498 (48 bytes)."""
    _fields_ = [("x", PolyRef), ("k", vp), ("pr", vp), ("n", i32), ("K", i32)]


class MulTableArgs(C.Structure):
    """args.cuh:500-506 (72 bytes)."""
    _fields_ = [("out", PolyRef), ("in_", PolyRef), ("t", vp), ("pr", vp), ("n", i32), ("K", i32)]


class MulAddArgs(C.Structure):
    """args.cuh:508-515 (104 bytes)."""
    _fields_ = [("m", MulTableArgs), ("y", PolyRef), ("sub", i32), ("pad", i32)]


class MulAddNArgs(C.Structure):
    """args.cuh:517-528 (328 bytes)."""
    _fields_ = [("out", PolyRef), ("y", PolyRef), ("x", PolyRef * 8), ("t", vp * 8), ("pr", vp), ("n", i32),
                ("K", i32), ("nterm", i32), ("lazy", i32)]


class RescaleArgs(C.Structure):
    """args.cuh:531-552 (152 bytes)."""
    _fields_ = [("x", PolyRef), ("tmp", PolyRef), ("A", vp), ("B", vp), ("As", vp), ("Bs", vp), ("qam", vp),
                ("qbm", vp), ("pr", vp), ("qinv_ab", u64), ("C_ab", u64), ("ca", u64), ("cb", u64), ("top", i32),
                ("nrows", i32), ("K", i32), ("ndrop", i32)]


class RescaleNttArgs(C.Structure):
    """args.cuh:554-563 (328 bytes)."""
    _fields_ = [("rs", RescaleArgs), ("ntt", NttArgs)]


class RescaleCombineArgs(C.Structure):
    """args.cuh:565-572 (80 bytes)."""
    _fields_ = [("x", PolyRef), ("tmp", PolyRef), ("alpha", vp), ("alphas", vp), ("pr", vp), ("n", i32), ("K", i32)]


class RescaleCombineToArgs(C.Structure):
    """args.cuh:574-579 (104 bytes)."""
    _fields_ = [("a", RescaleCombineArgs), ("out", PolyRef)]


EWM_MAX = 48


class EwManyArgs(C.Structure):
    """args.cuh:162-170."""
    _fields_ = [("out", vp * EWM_MAX), ("a", vp * EWM_MAX), ("b", vp * EWM_MAX), ("c", vp * EWM_MAX), ("pr", vp),
                ("n", i32), ("nrows", i32)]


class SubMulManyArgs(C.Structure):
    """args.cuh:172-182."""
    _fields_ = [("out", vp * EWM_MAX), ("a", vp * EWM_MAX), ("b", vp * EWM_MAX), ("t", vp), ("pr", vp), ("n", i32),
                ("nrows", i32)]


class EncryptArgs(C.Structure):
    """args.cuh:613-628 (64 bytes)."""
    _fields_ = [("c0", vp), ("c1", vp), ("s", vp), ("e", vp), ("m", vp), ("seed", vp), ("pr", vp), ("nonce", u32),
                ("nl", i32)]


class ModRaiseArgs(C.Structure):
    """args.cuh:665-676 (2136 bytes)."""
    _fields_ = [("x", vp), ("pr", vp), ("ct_stride", u64), ("part_stride", u64), ("qhatinv", u64 * 4),
                ("qhat", (u64 * 64) * 4), ("K", i32), ("d", i32), ("r0", i32), ("r1", i32), ("nparts", i32),
                ("pad", i32)]


class SmallIntTab(C.Structure):
    """args.cuh:678-697 (4552 bytes; lives in device memory)."""
    _fields_ = [("k", i32), ("nout", i32), ("nw", i32), ("nr", i32), ("divide", i32), ("pad", i32), ("q", u32 * 4),
                ("qinv", (u32 * 4) * 4), ("Qk", u32 * 8), ("Qkh", u32 * 8), ("R", u32 * 8), ("orow", i32 * 64),
                ("pow32", (u32 * 16) * 64)]


class SmallIntArgs(C.Structure):
    """args.cuh:698-709 (72 bytes)."""
    _fields_ = [("src", vp), ("out", vp), ("tab", vp), ("pr", vp), ("src_ct_stride", u64), ("src_part_stride", u64),
                ("ct_stride", u64), ("part_stride", u64), ("K", i32), ("nparts", i32)]


class SmallInt1Args(C.Structure):
    """args.cuh:890-907 (56 bytes)."""
    _fields_ = [("x", vp), ("pr", vp), ("ct_stride", u64), ("part_stride", u64), ("mc", u64), ("sh", i32),
                ("nrows", i32), ("K", i32), ("nparts", i32)]


class EncodeArgs(C.Structure):
    """args.cuh:595-611: device slot encoding (80 bytes)."""
    _fields_ = [("v", vp), ("a", vp), ("b", vp), ("c", vp), ("cmax", vp), ("out", vp), ("deg_factor", vp), ("pr", vp),
                ("scale", C.c_double), ("nl", i32), ("pad", i32)]


class KskExpandArgs(C.Structure):
    """args.cuh:306-323: KSKA rows out[d - d0][m][N] (48 bytes)."""
    _fields_ = [("out", vp), ("seed", vp), ("prime_ids", vp), ("pr", vp), ("nmod", i32), ("dnum", i32), ("d0", i32),
                ("pad", i32)]


class KskUnpackArgs(C.Structure):
    """args.cuh:656-663: packed key rows to dense rows (32 bytes)."""
    _fields_ = [("out", vp), ("in_", vp), ("row_words", u64), ("nrows", i32), ("bits", i32)]


class BconvArgs(C.Structure):
    """args.cuh:130-141: a batch of fast base-conversion jobs (56 bytes); jobs are 8 u32 words each (BconvJob: src_off,
    dst_off, nsrc, ntgt, pool_off, exact, prescaled, split)."""
    _fields_ = [("src", vp), ("dst", vp), ("jobs", vp), ("pool", vp), ("pr", vp), ("njobs", i32), ("max_tgt", i32),
                ("kind", i32), ("pad", i32)]


KS_ACC, KS_SUM = 4, 8  # KsArgs.c0_mode flags (args.cuh:207-210)

assert C.sizeof(KeyTab) == 40 and C.sizeof(CtsArgs) == 200 and C.sizeof(CtsRegenArgs) == 240
assert C.sizeof(KsArgs) == 176 and C.sizeof(KsKeyArgs) == 216 and C.sizeof(EpiArgs) == 72
assert C.sizeof(KsRegenArgs) == 312
assert C.sizeof(EwArgs) == 128 and C.sizeof(CoeffArgs) == 592 and C.sizeof(TensorSeededArgs) == 25656
assert C.sizeof(PolyRef) == 24 and C.sizeof(NttArgs) == 176 and C.sizeof(TensorArgs) == 192
assert C.sizeof(TensorYArgs) == 240 and C.sizeof(TensorSumArgs) == 2 * 24 + 2 * TSUM_MAX * 24 + 8 + 16
assert C.sizeof(MdEpiArgs) == 120 and C.sizeof(MdEpiToArgs) == 152 and C.sizeof(WsumArgs) == 256
assert C.sizeof(WsumKArgs) == 264 and C.sizeof(WsumMultiArgs) == 376 and C.sizeof(AddConstArgs) == 48
assert C.sizeof(MulTableArgs) == 72 and C.sizeof(MulAddArgs) == 104 and C.sizeof(MulAddNArgs) == 328
assert C.sizeof(RescaleArgs) == 152 and C.sizeof(RescaleNttArgs) == 328 and C.sizeof(RescaleCombineArgs) == 80
assert C.sizeof(RescaleCombineToArgs) == 104 and C.sizeof(EwManyArgs) == 4 * EWM_MAX * 8 + 16
assert C.sizeof(SubMulManyArgs) == 3 * EWM_MAX * 8 + 24
assert C.sizeof(ModRaiseArgs) == 2136 and C.sizeof(SmallIntTab) == 4552 and C.sizeof(SmallIntArgs) == 72
assert C.sizeof(SmallInt1Args) == 56 and C.sizeof(EncryptArgs) == 64
assert C.sizeof(EncodeArgs) == 80 and C.sizeof(KskExpandArgs) == 48 and C.sizeof(KskUnpackArgs) == 32 and C.sizeof(BconvArgs) == 56
assert C.sizeof(RowSet) == 16 and C.sizeof(PtDotArgs) == 128
assert C.sizeof(PackSplitArgs) == 64 and C.sizeof(PackDotArgs) == 120
assert C.sizeof(TensorMultiArgs) == (2 * TMULTI_OUT + 2 * TMULTI_OUT * TMULTI_PAIRS) * 24 + 8 + 24

_LAUNCHER = C.CFUNCTYPE(C.c_int, vp, vp)


def entry(name, log_n=16):
    """The table entry `name` of the ring 2^log_n as a callable f(args_pointer, stream) -> int."""
    base = LIB.pc_table_u32_logn(log_n)
    if not base:
        raise ValueError(f"no kernel table for log_n {log_n}")
    fp = C.c_void_p.from_address(base + 16 + 8 * ENTRIES.index(name)).value
    return _LAUNCHER(fp)


def call(name, args, stream=None, log_n=16):
    """Launch table entry `name` on `args` (a ctypes struct); returns the launcher's code (0, -1/-2/-3 or a HIP
    error)."""
    return entry(name, log_n)(C.addressof(args), None if stream is None else stream.h)
