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
