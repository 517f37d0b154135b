"""ctypes mirrors of the ABI-30 argument structs a Python caller fills to call the kernel table's CtS entries directly
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
    """args.cuh:284-294: a key set read in its stored form (40 bytes)."""
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
    """args.cuh:752-757: cts_fused with the baby keys through a KeyTab (240 bytes)."""
    _fields_ = [("cts", CtsArgs), ("key", KeyTab)]


class KsArgs(C.Structure):
    """args.cuh:211-228: the key-switch inner product (176 bytes)."""
    _fields_ = [("c1", vp), ("modup", vp), ("c0", vp), ("out0", vp), ("out1", vp), ("kb", vp), ("ka", vp),
                ("autok", vp), ("rows", vp), ("digit_of", vp), ("pmod", vp), ("pmods", vp), ("pr", vp),
                ("ct_stride", u64), ("mu_ct_stride", u64), ("mu_digit_stride", u64), ("out_ct_stride", u64),
                ("out_rot_stride", u64), ("key_digit_stride", u64), ("K", i32), ("R", i32), ("ndig", i32),
                ("c0_mode", i32), ("nq", i32), ("nrows", i32)]


class KsKeyArgs(C.Structure):
    """args.cuh:997-1003: ks_dot with the keys through a KeyTab (216 bytes)."""
    _fields_ = [("ks", KsArgs), ("key", KeyTab)]


class EpiArgs(C.Structure):
    """args.cuh:268-281: the fused relinearisation epilogue (72 bytes)."""
    _fields_ = [("dst", vp), ("conv", vp), ("binv", vp), ("binvs", vp), ("k", vp), ("part_stride", u64),
                ("dbl", i32), ("pad", i32), ("alpha", vp), ("alphas", vp)]


class KsRegenArgs(C.Structure):
    """args.cuh:299-307: the relinearisation dot with a regenerated key (312 bytes)."""
    _fields_ = [("ks", KsArgs), ("seed", vp), ("epi", EpiArgs), ("use_epi", i32), ("pad", i32), ("key", KeyTab),
                ("add", vp)]


KS_ACC, KS_SUM = 4, 8  # KsArgs.c0_mode flags (args.cuh:208-210)

assert C.sizeof(KeyTab) == 40 and C.sizeof(CtsArgs) == 200 and C.sizeof(CtsRegenArgs) == 240
assert C.sizeof(KsArgs) == 176 and C.sizeof(KsKeyArgs) == 216 and C.sizeof(EpiArgs) == 72
assert C.sizeof(KsRegenArgs) == 312

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
