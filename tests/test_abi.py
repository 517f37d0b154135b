"""The C-ABI boundary, checked without a GPU: the library loads, exports every function include/pc_hip.h declares,
its tables carry the reference's header {abi 30, word 4 bytes, Barrett64, log_n} (crates/pc-kernels/src/table.rs:101-112)
and every launcher rejects a null argument struct with -1 before touching the device (args.cuh:1036)."""
import ctypes as C

import pytest

import perseus_amd as pa
from perseus_amd._lib import LIB
from tests import twin


class KernelTable(C.Structure):
    _fields_ = [("abi", C.c_uint32), ("word_bytes", C.c_uint32), ("mm", C.c_uint32), ("log_n", C.c_uint32)] + [
        (f"f{i}", C.c_void_p) for i in range(52)]


def table(logn=None):
    p = LIB.pc_table_u32_barrett64() if logn is None else LIB.pc_table_u32_logn(logn)
    assert p
    return KernelTable.from_address(p)


def test_every_declared_symbol_is_exported():
    names = pa.header_functions()
    assert len(names) >= 50
    for n in names:
        assert hasattr(LIB, n), n


def test_table_headers():
    t = table()
    assert (t.abi, t.word_bytes, t.mm, t.log_n) == (30, 4, 0, 16)
    assert C.sizeof(KernelTable) == 16 + 52 * 8
    for logn in range(12, 17):
        t = table(logn)
        assert (t.abi, t.word_bytes, t.mm, t.log_n) == (30, 4, 0, logn)
    assert not LIB.pc_table_u32_logn(11) and not LIB.pc_table_u32_logn(17)


def test_null_arguments_are_rejected():
    launcher = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_void_p)
    for logn in (12, 14, 16):
        t = table(logn)
        for i in range(52):
            f = launcher(getattr(t, f"f{i}"))
            assert f(None, None) == -1, i


def test_chains_match_the_oracle_primes():
    for name, (bits, logn, n) in {"c1": (30, 14, 16), "c2": (31, 16, 40), "c3": (31, 16, 36)}.items():
        c = pa.preset(name)
        assert c.primes == twin.descending_primes(bits, 2 << logn, n)
        assert all(p < (1 << 31) and (p - 1) % (2 << logn) == 0 for p in c.primes)
    c3 = pa.preset("c3")
    assert (len(c3.q), len(c3.p), c3.dnum, c3.alpha) == (30, 6, 3, 10)
    c1 = pa.preset("c1")
    assert (len(c1.q), len(c1.p), c1.dnum, c1.alpha, c1.logn) == (12, 4, 3, 4, 14)


def test_entry_names_follow_the_header():
    """perseus_amd.abi.ENTRIES is KernelTable's field order (args.cuh:1037-1097) as include/pc_hip.h declares it."""
    import re
    from perseus_amd import abi
    text = open(pa._lib.HEADER).read()
    body = text[text.index("typedef struct KernelTable"):text.index("} KernelTable;")]
    assert re.findall(r"\(\*(\w+)\)", body) == abi.ENTRIES


def test_cts_launchers_reject_out_of_range_arguments():
    """The CtS launchers' argument checks (crates/pc-kernels/kernels/cts.cuh:480-524 launch_any / launch_regen, plus
    this kernel's own range), all decided before any device call."""
    from perseus_amd import abi
    a = abi.CtsArgs()
    a.K, a.B, a.G, a.ndig, a.nrows, a.kmax, a.npts, a.ptw, a.enc = 1, 3, 2, 3, 4, 1, 6, 4096, 0xFFFFFFFF
    fused = lambda: abi.call("cts_fused", a, log_n=12)  # noqa: E731
    a.G = 3
    assert fused() == -1                       # three giant steps outside the pair form
    a.G, a.pair_cts = 2, 2
    assert fused() == -1                       # the pair layout is a regen-form feature
    a.pair_cts, a.ndig = 0, 7
    assert fused() == -1                       # more than 6 digits
    a.ndig, a.x0, a.kmax = 3, 0x1000, 2
    assert fused() == -1                       # x0 with groups of ciphertexts
    a.x0, a.kmax, a.K = None, 1, 0
    assert fused() == 0                        # nothing to do
    a.K = 1
    assert fused() == -1                       # null row list
    r = abi.CtsRegenArgs()
    r.cts.K, r.cts.B, r.cts.G, r.cts.ndig, r.cts.nrows, r.cts.kmax, r.cts.ptw = 1, 3, 4, 3, 4, 1, 4096
    r.cts.enc, r.cts.npts = 0xFFFFFFFF, 12
    regen = lambda: abi.call("cts_fused_regen", r, log_n=12)  # noqa: E731
    r.key.bits = 33
    assert regen() == -1                       # packed width above 32
    r.key.bits = 0
    assert regen() == -1                       # four giant steps need the pair layout
    r.cts.pair_cts, r.cts.G = 2, 5
    assert regen() == -1                       # at most four in it
    r.cts.G, r.cts.K = 4, 2
    assert regen() == -1                       # the pair layout is for one ciphertext
    r.cts.K, r.cts.B = 1, 65
    assert regen() == -1                       # at most 64 baby steps
    r.cts.B, r.cts.x0 = 3, 0x1000
    assert regen() == -1                       # x0 outside the four-giant-step form only
    r.cts.x0 = None
    assert regen() == -1                       # null row list
    b = abi.CtsRegenArgs()
    c = b.cts
    c.K, c.B, c.G, c.ndig, c.nrows, c.kmax, c.npts = 1, 2, 2, 3, 4, 1, 2
    c.rows = c.pr = c.x = c.res = c.digit_of = c.pmod = c.pmods = c.pts = c.kinv = c.modup = 0x1000
    b.key.kb = b.key.seed = 0x1000
    b.key.nregen = 3
    c.enc, c.ptw = 0x7F000003, 511
    assert abi.call("cts_fused_regen", b, log_n=12) == -1   # a block-constant diagonal needs N >> 3 words
    c.enc, c.ptw = 0x3FF, 1023
    assert abi.call("cts_fused_regen", b, log_n=12) == -1   # a periodic one (o & enc) needs enc + 1
    c.ptw, c.ct_stride = 1024, 2 * 8 * 4096 + 1
    assert abi.call("cts_fused_regen", b, log_n=12) == -2   # rows of whole 16-byte groups


def test_dot_launchers_reject_out_of_range_arguments():
    """ks_dot_regen's checks (crates/pc-host/src/ks.rs:267-280) and ks_dot's refusal of the summed rotations
    (KS_SUM: -3, crates/pc-host/src/ks.rs:151-153), decided before any device call."""
    from perseus_amd import abi
    g = abi.KsRegenArgs()
    g.ks.K, g.ks.nrows, g.ks.ndig = 1, 2, 3
    g.key.kb, g.key.bits = 0x1000, 33
    assert abi.call("ks_dot_regen", g, log_n=12) == -1     # packed width above 32
    g.key.bits, g.add = 0, 0x1000
    assert abi.call("ks_dot_regen", g, log_n=12) == -1     # `add` outside the fused epilogue
    g.add, g.ks.K = None, 5
    assert abi.call("ks_dot_regen", g, log_n=12) == -2     # more than 4 ciphertexts
    g.ks.K = 0
    assert abi.call("ks_dot_regen", g, log_n=12) == 0      # nothing to do
    g.ks.K = 1
    assert abi.call("ks_dot_regen", g, log_n=12) == -1     # null row list
    k = abi.KsArgs()
    k.c0_mode, k.K = abi.KS_SUM, 1
    assert abi.call("ks_dot", k, log_n=12) == -3           # the summed rotations: ks_dot_key only
    kk = abi.KsKeyArgs()
    kk.ks.c0_mode, kk.ks.K = abi.KS_SUM, 5
    assert abi.call("ks_dot_key", kk, log_n=12) == -2      # K > 4


def test_em_launchers_reject_out_of_range_arguments():
    """The EvalMod / rescale launchers' count checks (crates/pc-kernels/kernels/em.cuh:580-692, rescale.cuh:211-263)
    and null operands, all decided before any device call."""
    from perseus_amd import abi
    assert abi.call("wsum_multi", abi.WsumMultiArgs(), log_n=12) == -1      # nout 0
    m = abi.MulAddArgs()
    m.sub = 3
    assert abi.call("mul_add", m, log_n=12) == -1                           # sub outside 0..2
    n = abi.MulAddNArgs()
    n.nterm = 9
    assert abi.call("mul_add_n", n, log_n=12) == -1                         # more than 8 terms
    s = abi.TensorSumArgs()
    s.npairs = 17
    assert abi.call("tensor_sum", s, log_n=12) == -1                        # more than 16 pairs
    r = abi.RescaleArgs()
    r.ndrop = 3
    assert abi.call("rescale_coef", r, log_n=12) == -1                      # one or two primes only
    rf = abi.RescaleNttArgs()
    rf.rs.ndrop = 1
    assert abi.call("rescale_fwd", rf, log_n=12) == -1                      # the pipeline drops two
    assert abi.call("ew_many", abi.EwManyArgs(), log_n=12) == -1            # n 0
    assert abi.call("tensor_y", abi.TensorYArgs(), log_n=12) == -1          # no y constant
    assert abi.call("md_epilogue", abi.MdEpiArgs(), log_n=12) == -1         # null operands
    w = abi.WsumArgs()
    w.nsrc = 9
    assert abi.call("wsum", w, log_n=12) == -1                              # more than 8 sources
    t = abi.TensorArgs()
    assert abi.call("tensor", t, log_n=12) == -1                            # null outputs
    # pt_dot: diagonal indices outside the rows of ptw words (fake, never dereferenced operand addresses)
    for enc, ptw in ((0xFFFFFFFF, 4095), (0x7F000004, 255), (0x3FF, 1023), (0x7F000020, 1 << 12), (0xFFFFFFFF, 0)):
        p = abi.PtDotArgs()
        p.rot = abi.PolyRef(64, 0, 0)
        p.res = abi.PolyRef(64, 0, 0)
        p.pts, p.pr = 64, 64
        p.rs = abi.RowSet(1, 0, 1, 0)
        p.npts, p.bstep, p.gstep, p.K, p.ptw, p.enc = 1, 1, 1, 1, ptw, enc
        assert abi.call("pt_dot", p, log_n=12) == -1


def test_raise_launchers_reject_out_of_range_arguments():
    """The raise launchers' checks (crates/pc-kernels/kernels/bts.cuh:192-218), decided before any device call."""
    from perseus_amd import abi
    m = abi.ModRaiseArgs()
    m.d, m.r0, m.r1, m.nparts, m.K = 5, 5, 8, 1, 1
    assert abi.call("mod_raise", m, log_n=12) == -1      # more than four sources
    m.d, m.r0 = 2, 1
    assert abi.call("mod_raise", m, log_n=12) == -1      # a target row among the sources
    m.r0, m.r1 = 2, 65
    assert abi.call("mod_raise", m, log_n=12) == -1      # past 64 rows
    s = abi.SmallIntArgs()
    s.nparts, s.K = 3, 1
    assert abi.call("small_int", s, log_n=12) == -1      # three parts
    s1 = abi.SmallInt1Args()
    s1.sh, s1.nrows, s1.K, s1.nparts = 0, 1, 1, 1
    assert abi.call("small_int1", s1, log_n=12) == -1    # shift 0
    s1.sh, s1.nrows = 3, 65
    assert abi.call("small_int1", s1, log_n=12) == -1    # past 64 rows


def test_encrypt_launcher_rejects_null_operands():
    from perseus_amd import abi
    a = abi.EncryptArgs()
    a.nl = 2
    assert abi.call("encrypt", a, log_n=12) == -1


def test_pt_dot_launcher_checks():
    from perseus_amd import abi
    a = abi.PtDotArgs()
    a.K = 9
    assert abi.call("pt_dot", a, log_n=12) == -1    # more than 8 ciphertexts
    a.K = 1
    assert abi.call("pt_dot", a, log_n=12) == -1    # null operands


def test_pack_launcher_checks():
    """pack_split / pack_dot (crates/pc-kernels/kernels/ks.cuh:949-963): sub a power of two in 2..16, nq <= nrows."""
    from perseus_amd import abi
    a = abi.PackSplitArgs()
    a.K, a.nq, a.nrows = 1, 2, 4
    for sub in (1, 3, 32):
        a.sub = sub
        assert abi.call("pack_split", a, log_n=12) == -1
    a.sub, a.nq = 4, 5
    assert abi.call("pack_split", a, log_n=12) == -1
    d = abi.PackDotArgs()
    d.K, d.sub, d.nq, d.nrows = 1, 4, 2, 4
    assert abi.call("pack_dot", d, log_n=12) == -1   # null operands


def test_tensor_multi_launcher_checks():
    from perseus_amd import abi
    a = abi.TensorMultiArgs()
    a.nout, a.npairs = 5, 1
    assert abi.call("tensor_multi", a, log_n=12) == -1   # more than 4 outputs
    a.nout, a.npairs = 1, 33
    assert abi.call("tensor_multi", a, log_n=12) == -1   # more than 32 pairs


def test_struct_mirrors_match_the_header_sizes():
    """the ctypes mirrors of the argument structs have the sizes include/pc_hip.h asserts (args.cuh's layouts)"""
    from perseus_amd import abi
    sizes = {"PolyRef": 24, "EwArgs": 128, "CoeffArgs": 592, "TensorSeededArgs": 25656, "SpruFftArgs": 32,
             "SpruScatterArgs": 56, "KskExpandArgs": 48, "KskUnpackArgs": 32, "BconvArgs": 56, "KsArgs": 176,
             "KsKeyArgs": 216, "KsRegenArgs": 312, "KeyTab": 40}
    for name, size in sizes.items():
        assert C.sizeof(getattr(abi, name)) == size, name
