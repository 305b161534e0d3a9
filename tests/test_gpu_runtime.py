"""Runtime exports on the GPU: the byte fill behind eng_memset_async and the
stream hold eng_stream_delay, through the C-ABI.

eng_memset_async is a fill kernel (not hipMemsetAsync), so it may be captured
into a HIP graph: the graph test replays it several times with eager work in
between and checks every replay. The expected bytes are plain numpy.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("offset,nbytes,value", [
    (0, 1, 0x5A), (1, 15, 0xFF), (3, 17, 0x01), (0, 16, 0x80), (7, 4096 + 9, 0x3C),
    (13, (1 << 20) + 77, 0xA5), (0, 3 * (1 << 22), 0x00), (5, 0, 0x11)])
def test_memset_async_fills_exact_bytes(gpu, offset, nbytes, value):
    total = offset + nbytes + 64
    buf = gpu.empty(total, np.uint8)
    s = gpu.stream()
    try:
        gpu.call("eng_memset", buf.ptr, 0xEE, total)
        gpu.call("eng_memset_async", buf.ptr + offset, value | 0x100 * 7, nbytes, s.handle)
        s.sync()
        got = buf.download()
        want = np.full(total, 0xEE, np.uint8)
        want[offset:offset + nbytes] = value
        assert np.array_equal(got, want)
    finally:
        s.destroy()
        buf.free()


def test_memset_async_rejects_null(gpu):
    s = gpu.stream()
    try:
        rc = gpu.lib.eng_memset_async(None, 0, 16, s.handle)
        assert rc == 1 and "null" in gpu.last_error()
        assert gpu.lib.eng_memset_async(None, 0, 0, s.handle) == 0   # zero bytes: no-op
    finally:
        s.destroy()


def test_memset_async_in_a_graph_replays(gpu):
    n = 100_003
    buf = gpu.empty(n + 3, np.uint8)
    other = gpu.empty(4096, np.uint8)
    s = gpu.stream()
    graph = None
    try:
        gpu.call("eng_memset_async", buf.ptr + 3, 0x42, n, s.handle)   # eager first
        s.sync()
        graph = gpu.graph(s)
        with graph:
            gpu.call("eng_memset_async", buf.ptr + 3, 0x42, n, s.handle)
            gpu.call("eng_memset_async", other.ptr, 0x17, 4096, s.handle)
        for rep in range(4):
            gpu.call("eng_memset", buf.ptr, 0x00, n + 3)
            gpu.call("eng_memset", other.ptr, 0x00, 4096)
            gpu.call("eng_memset_async", other.ptr, 0x99, 100, s.handle)   # eager work between
            s.sync()
            graph.launch()
            s.sync()
            got = buf.download()
            assert np.all(got[:3] == 0), f"replay {rep}: bytes before the fill changed"
            assert np.all(got[3:] == 0x42), f"replay {rep}"
            assert np.all(other.download() == 0x17), f"replay {rep}"
    finally:
        if graph is not None:
            graph.destroy()
        s.destroy()
        buf.free()
        other.free()


def test_stream_delay_holds_the_stream(gpu):
    s = gpu.stream()
    e0, e1 = gpu.event(), gpu.event()
    try:
        for us in (0, 200, 2000):
            e0.record(s)
            gpu.call("eng_stream_delay", s.handle, us)
            e1.record(s)
            e1.sync()
            ms = e0.elapsed_ms(e1)
            assert ms >= 0.95 * us / 1000.0, (us, ms)
            assert ms < us / 1000.0 + 5.0, (us, ms)
        # Work queued behind the hold runs after it, in order.
        y = gpu.empty(1024, np.uint8)
        gpu.call("eng_memset", y.ptr, 0, 1024)
        gpu.call("eng_stream_delay", s.handle, 1000)
        gpu.call("eng_memset_async", y.ptr, 0x7E, 1024, s.handle)
        s.sync()
        assert np.all(y.download() == 0x7E)
        y.free()
    finally:
        e0.destroy(), e1.destroy()
        s.destroy()


def test_stream_delay_bounds(gpu):
    s = gpu.stream()
    try:
        rc = gpu.lib.eng_stream_delay(s.handle, ctypes.c_uint(1_000_001))
        assert rc == 1 and "at most 1000000" in gpu.last_error()
    finally:
        s.destroy()
