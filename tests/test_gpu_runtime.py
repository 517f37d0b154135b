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


def test_capture_beside_cyclic_garbage_holding_device_buffers():
    """Device buffers whose last references sit in reference cycles are freed by Python's cyclic collector whenever it
    runs, and a free inside a stream capture would invalidate it: pa.Graph collects before it begins and holds the
    collector off until the capture ends. The captured work allocates far past the collector's thresholds; the graph
    is built and its replay copies the words."""
    say("[graph] capture beside cyclic garbage that holds device buffers")
    st = pa.Stream()
    n = 1 << 16
    src = pa.DevBuf.from_array(np.arange(n, dtype=np.uint32))
    dst = pa.DevBuf(n)
    for _ in range(8):
        cyc = [pa.DevBuf(1024)]
        cyc.append(cyc)  # a cycle: only the collector frees its buffer
    del cyc

    def work():
        junk = [[i] for i in range(200000)]
        assert LIB.pc_hip_memcpy_dtod(dst.ptr, src.ptr, 4 * n, st.h) == 0
        del junk

    g = pa.Graph(st, work)
    g.launch(st)
    st.sync()
    assert (dst.download() == np.arange(n, dtype=np.uint32)).all()


def test_device_queries_of_device_open():
    """What crates/pc-cuda/src/device.rs:63-158 (Device::open, sm_count, clusters, mem_info, profiler) reads."""
    say("[runtime] versions, attributes, memory info, profiler range, priority range")
    rt, dr = C.c_int(0), C.c_int(0)
    assert LIB.pc_hip_runtime_version(C.byref(rt)) == 0 and rt.value > 0
    assert LIB.pc_hip_driver_version(C.byref(dr)) == 0 and dr.value > 0
    v = C.c_int(-1)
    assert LIB.pc_hip_device_attribute(C.byref(v), 16, 0) == 0
    assert v.value == 256, v.value  # MI355X: 256 compute units
    assert LIB.pc_hip_device_attribute(C.byref(v), 75, 0) == 0 and v.value == 9
    assert LIB.pc_hip_device_attribute(C.byref(v), 76, 0) == 0 and v.value == 5
    assert LIB.pc_hip_device_attribute(C.byref(v), 0x10000, 0) == 0 and v.value == 0
    assert LIB.pc_hip_device_attribute(C.byref(v), 0x10001, 0) == 0 and v.value == 0x950
    assert LIB.pc_hip_device_attribute(C.byref(v), 13, 0) == 0 and 1_000_000 <= v.value <= 4_000_000  # kHz
    assert LIB.pc_hip_device_attribute(C.byref(v), 12345, 0) != 0
    assert LIB.pc_hip_device_attribute(C.byref(v), 16, 99) != 0  # no such device
    # the failure is reported once, by its return code: the thread's last error is clear for the next launch's check
    assert LIB.pc_hip_last_error() == 0
    free, total = C.c_size_t(0), C.c_size_t(0)
    assert LIB.pc_hip_mem_get_info(C.byref(free), C.byref(total)) == 0
    assert 0 < free.value <= total.value and total.value > (250 << 30)  # 288 GB of HBM3E
    buf = pa.DevBuf(1 << 28)  # 1 GiB: free memory drops by about that much
    free2 = C.c_size_t(0)
    assert LIB.pc_hip_mem_get_info(C.byref(free2), C.byref(total)) == 0
    assert free.value - free2.value >= (1 << 30) - (64 << 20), (free.value, free2.value)
    del buf
    assert LIB.pc_hip_profiler_start() == 0 and LIB.pc_hip_profiler_stop() == 0
    lo, hi = C.c_int(-7), C.c_int(-7)
    assert LIB.pc_hip_stream_priority_range(C.byref(lo), C.byref(hi)) == 0 and (lo.value, hi.value) == (0, 0)
    assert LIB.pc_hip_error_name(1) and LIB.pc_hip_error_name(-1) == b"PC_LAUNCH_ARGS"


def test_events_with_flags_and_a_priority_stream():
    """Event::new (ordering only: no elapsed time) and Event::timing (crates/pc-cuda/src/stream.rs:133-147) on a
    stream made by Stream::high_priority's call, ordering a copy between two streams."""
    say("[runtime] event flags: ordering-only and timing events across two streams")
    s1, s2 = C.c_void_p(), C.c_void_p()
    assert LIB.pc_hip_stream_create_with_priority(C.byref(s1), -1) == 0
    assert LIB.pc_hip_stream_create(C.byref(s2)) == 0
    ev_order, t0, t1 = C.c_void_p(), C.c_void_p(), C.c_void_p()
    assert LIB.pc_hip_event_create_flags(C.byref(ev_order), 2) == 0
    assert LIB.pc_hip_event_create_flags(C.byref(t0), 0) == 0
    assert LIB.pc_hip_event_create_flags(C.byref(t1), 0) == 0
    assert LIB.pc_hip_event_create_flags(C.byref(C.c_void_p()), 4) != 0  # unknown flag bits
    n = 1 << 22
    src = pa.DevBuf.from_array(np.arange(n, dtype=np.uint32))
    mid, dst = pa.DevBuf(n), pa.DevBuf(n)
    assert LIB.pc_hip_event_record(t0, s1) == 0
    assert LIB.pc_hip_memcpy_dtod(mid.ptr, src.ptr, 4 * n, s1) == 0
    assert LIB.pc_hip_event_record(ev_order, s1) == 0
    assert LIB.pc_hip_event_record(t1, s1) == 0
    assert LIB.pc_hip_stream_wait_event(s2, ev_order) == 0
    assert LIB.pc_hip_memcpy_dtod(dst.ptr, mid.ptr, 4 * n, s2) == 0
    assert LIB.pc_hip_stream_sync(s2) == 0 and LIB.pc_hip_event_sync(t1) == 0
    assert (dst.download() == np.arange(n, dtype=np.uint32)).all()
    ms = C.c_float(-1)
    assert LIB.pc_hip_event_elapsed_ms(C.byref(ms), t0, t1) == 0 and ms.value >= 0
    for e in (ev_order, t0, t1):
        assert LIB.pc_hip_event_destroy(e) == 0
    for s in (s1, s2):
        assert LIB.pc_hip_stream_destroy(s) == 0


def test_valu_probe_runs_and_rejects_bad_arguments():
    """pcx_valu_probe: every instruction form runs to completion on a small grid; a bad kind or size is refused"""
    out = pa.DevBuf(1024)
    st = pa.Stream()
    for kind in range(7):
        assert LIB.pcx_valu_probe(kind, 4, 8, out.ptr, st.h) == 0
    st.sync()
    assert LIB.pcx_valu_probe(7, 4, 8, out.ptr, st.h) == -1
    assert LIB.pcx_valu_probe(0, 0, 8, out.ptr, st.h) == -1
    assert LIB.pcx_valu_probe(0, 4, 0, out.ptr, st.h) == -1
    assert LIB.pcx_valu_probe(0, 4, 8, None, st.h) == -1
