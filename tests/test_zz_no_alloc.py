"""eng_rmsnorm_linear_f16w_noalloc: the allocation-free variant of
eng_rmsnorm_linear_f16w (split-K partial sums in a static device buffer).

Through the C-ABI: each call must equal eng_rmsnorm_linear_f16w's output bit
for bit (same kernels and configuration: split-K GEMV passes up to 4 rows,
the few-row MFMA kernel from 5) and the oracle within the derived bound, on
consecutive calls whose second input is smaller (the static buffer keeps the
last call's contents), on the null stream and a created stream, at the decode
and small-batch row counts. Shapes past the limits fail with a message and
write nothing."""

from __future__ import annotations

import numpy as np
import pytest

import helpers

pytestmark = pytest.mark.gpu
EPS = 1e-5


def _case(gpu, rng, M, N, K):
    W16 = gpu.f32_to_f16((0.02 * rng.standard_normal((K, N))).astype(np.float32))
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    return W16, g, x


def _run(gpu, name, dW, dg, dx, M, N, K, stream):
    y = gpu.empty((M, N), np.float32)
    gpu.call("eng_memset", y.ptr, 0xFF, y.nbytes)
    gpu.call(name, dx.ptr, None if dg is None else dg.ptr, dW.ptr, y.ptr, M, N, K, EPS, stream)
    gpu.sync()
    out = y.download()
    y.free()
    return out


@pytest.mark.parametrize("use_stream", [False, True])
def test_noalloc_matches_the_allocating_entry_on_consecutive_calls(gpu, orc, use_stream):
    rng = np.random.default_rng(31)
    s = gpu.stream() if use_stream else None
    h = s.handle if s else None
    try:
        # larger first, then smaller: the second call reads a buffer the first
        # one filled further
        for M, N, K in ((16, 11008, 4096), (4, 11008, 4096), (1, 4096, 4096), (16, 2048, 1024),
                        (5, 1000, 776), (3, 1000, 777), (1, 512, 256)):
            W16, g, x = _case(gpu, rng, M, N, K)
            dW, dg, dx = gpu.upload(W16), gpu.upload(g), gpu.upload(x)
            want = _run(gpu, "eng_rmsnorm_linear_f16w", dW, dg, dx, M, N, K, h)
            got = _run(gpu, "eng_rmsnorm_linear_f16w_noalloc", dW, dg, dx, M, N, K, h)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
                f"M={M} N={N} K={K}: noalloc result differs from eng_rmsnorm_linear_f16w"
            y64 = helpers.as_f64(orc.rmsnorm_linear(x, g, W16, EPS))
            derived, _ = helpers.rmsnorm_linear_bounds(x, g, W16, y64, K)
            helpers.assert_within(got, y64, derived, f"noalloc M={M} N={N} K={K} vs oracle")
            for d in (dW, dg, dx):
                d.free()
    finally:
        if s:
            s.destroy()


def test_noalloc_without_gain(gpu, orc):
    rng = np.random.default_rng(32)
    M, N, K = 2, 4096, 2048
    W16, _, x = _case(gpu, rng, M, N, K)
    dW, dx = gpu.upload(W16), gpu.upload(x)
    want = _run(gpu, "eng_rmsnorm_linear_f16w", dW, None, dx, M, N, K, None)
    got = _run(gpu, "eng_rmsnorm_linear_f16w_noalloc", dW, None, dx, M, N, K, None)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_noalloc_limits_and_zero_sizes(gpu):
    y = gpu.empty((17, 64), np.float32)
    x = gpu.empty((17, 64), np.float32)
    W = gpu.empty((64, 64), np.uint16)
    gpu.call("eng_memset", y.ptr, 0x7F, y.nbytes)
    rc = gpu.status("eng_rmsnorm_linear_f16w_noalloc", x.ptr, None, W.ptr, y.ptr, 17, 64, 64,
                    EPS, None)
    assert rc == 1 and "at most 16 rows" in gpu.last_error()
    rc = gpu.status("eng_rmsnorm_linear_f16w_noalloc", x.ptr, None, None, y.ptr, 1, 64, 64,
                    EPS, None)
    assert rc == 1 and "null device pointer" in gpu.last_error()
    rc = gpu.status("eng_rmsnorm_linear_f16w_noalloc", x.ptr, None, W.ptr, y.ptr, 1, 64, 64,
                    -1.0, None)
    assert rc == 1 and "eps must be non-negative" in gpu.last_error()
    for M, N, K in ((0, 64, 64), (1, 0, 64), (1, 64, 0)):
        gpu.call("eng_rmsnorm_linear_f16w_noalloc", x.ptr, None, W.ptr, y.ptr, M, N, K, EPS, None)
    gpu.sync()
    assert (y.download().view(np.uint32) == 0x7F7F7F7F).all(), "a zero-size call wrote output"


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (4, 11008, 4096), (16, 2048, 1024),
                                   (5, 1000, 776)])
def test_noalloc_first_call_under_capture_on_a_fresh_stream(gpu, M, N, K):
    """The first call on a new stream is made inside a HIP graph capture, where
    a stream scratch arena cannot be grown: the capture succeeds only if the
    entry point leases none. Every replay must equal the allocating entry's
    eager result (computed on another stream) bit for bit."""
    rng = np.random.default_rng(33 + M)
    W16, g, x = _case(gpu, rng, M, N, K)
    dW, dg, dx = gpu.upload(W16), gpu.upload(g), gpu.upload(x)
    want = _run(gpu, "eng_rmsnorm_linear_f16w", dW, dg, dx, M, N, K, None)
    y = gpu.empty((M, N), np.float32)
    s = gpu.stream()
    graph = None
    try:
        graph = gpu.graph(s)
        with graph:
            gpu.call("eng_rmsnorm_linear_f16w_noalloc", dx.ptr, dg.ptr, dW.ptr, y.ptr, M, N, K,
                     EPS, s.handle)
        for rep in range(3):
            gpu.call("eng_memset", y.ptr, 0xFF, y.nbytes)
            graph.launch()
            s.sync()
            got = y.download()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
                f"replay {rep}: M={M} N={N} K={K} differs from eng_rmsnorm_linear_f16w"
    finally:
        if graph is not None:
            graph.destroy()
        s.destroy()
        for d in (dW, dg, dx, y):
            d.free()
