"""The runtime FFI's fill (pc_hip_memset, a kernel in place of cudaMemsetAsync): every byte of the range set to the
value's low byte and none outside it, at unaligned heads and tails and sizes from 1 byte; and inside a captured HIP
graph, replayed several times with eager writes between the replays, each replay checked."""
import ctypes as C
import sys

import numpy as np
import pytest

import perseus_amd as pa
from perseus_amd._lib import LIB

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bytes_of(buf):
    return buf.download().view(np.uint8)


@pytest.mark.parametrize("off,size,val", [(0, 1, 0x5A), (3, 13, 0xFF), (1, 16, 0x01), (7, 4096 + 9, 0x80),
                                          (16, 1 << 20, 0x00), (5, (1 << 22) + 3, 0x3C), (0, 0, 0x77)])
def test_memset_ranges(off, size, val):
    say(f"[memset] offset {off} bytes {size} value {val:#x}")
    st = pa.Stream()
    words = (off + size + 64) // 4 + 1
    rng = np.random.default_rng(off + size)
    init = rng.integers(0, 1 << 32, words, dtype=np.uint64).astype(np.uint32)
    buf = pa.DevBuf.from_array(init)
    assert LIB.pc_hip_memset(C.c_void_p(buf.ptr.value + off), val | 0x1200, size, st.h) == 0
    st.sync()
    want = init.view(np.uint8).copy()
    want[off: off + size] = val
    assert (bytes_of(buf) == want).all()


def test_memset_in_a_captured_graph():
    say("[memset] captured in a graph with a copy, replayed 4 times with eager writes between")
    st = pa.Stream()
    n = (1 << 18) + 5
    a = pa.DevBuf(n)
    b = pa.DevBuf(n)
    src = pa.DevBuf.from_array(np.arange(n, dtype=np.uint32))

    def work():
        assert LIB.pc_hip_memset(C.c_void_p(a.ptr.value + 4), 0xAB, 4 * (n - 2) + 1, st.h) == 0
        assert LIB.pc_hip_memcpy_dtod(b.ptr, src.ptr, 4 * n, st.h) == 0
        assert LIB.pc_hip_memset(C.c_void_p(b.ptr.value + 8), 0, 12, st.h) == 0

    g = pa.Graph(st, work)
    rng = np.random.default_rng(3)
    for rep in range(4):
        junk = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
        a.upload(junk, st)
        b.upload(junk[::-1].copy(), st)
        g.launch(st)
        st.sync()
        wa = junk.view(np.uint8).copy()
        wa[4: 4 + 4 * (n - 2) + 1] = 0xAB
        assert (bytes_of(a) == wa).all(), rep
        wb = np.arange(n, dtype=np.uint32)
        wb[2:5] = 0
        assert (b.download() == wb).all(), rep
